// Generic FlashAttention-2 forward for the one shape the MFMA kernels do not take: fp32
// Q/K/V (computed in fp32 throughout) at head dim 16 (fp32 at 32 to 256 runs on the fp32 MFMA
// kernel, 16-bit storage on the 16-bit MFMA kernel).  The template is written for any storage
// type and head dim, but only <float, 16> is instantiated.  This is the role of the reference's SIMT kernel
// attn_fwd_kernel (csrc/flash_attn.cu:54-187) and of its Triton kernel's other head
// dims (fused_attn/triton_fwd.py:210-222): same semantics as the MFMA prefill kernel
// (bottom-right causal mask, GQA, varlen, natural-log LSE, zero rows without keys).
//
// A workgroup of 256 threads owns 64 queries of one q-head; four threads share a
// query and hold D/4 of its elements of q and of the output accumulator.  K/V
// tiles of BN keys are converted to fp32 into LDS; for each key the four partial
// dot products are combined with two lane swaps, and the softmax is online per tile
// (one rescale per tile, not per key).  Scores are kept in the log2 domain.
#include <float.h>

#include "fa_device.hpp"
#include "fa_internal.hpp"

namespace fa {

template <class T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ float to_f32<__bf16>(__bf16 x) {
  return (float)x;
}
template <>
__device__ __forceinline__ float to_f32<_Float16>(_Float16 x) {
  return (float)x;
}

template <class T, int D>
__global__ void __launch_bounds__(256) attn_generic_kernel(const TileArgs a) {
  constexpr int BM = 64;              // queries per workgroup
  constexpr int TPR = 4;              // threads per query
  constexpr int DPT = D / TPR;        // elements per thread
  constexpr int BN = D >= 256 ? 16 : 32;  // keys per LDS tile
  constexpr int LDK = D + 4;          // fp32 row pitch in LDS (16-byte aligned rows)
  constexpr float NEG_INF = -__builtin_inff();
  static_assert(D % 16 == 0 && DPT % 4 == 0, "head dim");

  __shared__ __align__(16) float ks[BN * LDK];
  __shared__ __align__(16) float vs[BN * LDK];

  const int nrb = a.n_rowblk;
  const int rb = (int)blockIdx.x % nrb;
  const int bh = (int)blockIdx.x / nrb;
  const int hq = bh % a.hq;
  const int b = bh / a.hq;
  const int kvh = hq / a.group;

  int seq_q = a.nq, seq_k = a.nk;
  int64_t qtok0 = 0, ktok0 = 0;
  if (a.varlen) {
    const int qs = __builtin_amdgcn_readfirstlane(a.cu_q[b]);
    const int ks0 = __builtin_amdgcn_readfirstlane(a.cu_k[b]);
    seq_q = __builtin_amdgcn_readfirstlane(a.cu_q[b + 1]) - qs;
    seq_k = __builtin_amdgcn_readfirstlane(a.cu_k[b + 1]) - ks0;
    qtok0 = qs;
    ktok0 = ks0;
  }
  const int r0 = rb * BM;
  if (r0 >= seq_q) return;  // uniform over the workgroup
  const int offset = seq_k - seq_q;  // bottom-right causal alignment (reference.py:24-33)
  int khi = seq_k;
  if (a.causal) khi = min(khi, min(r0 + BM, seq_q) - 1 + offset + 1);

  const int tid = (int)threadIdx.x;
  const int qi = r0 + tid / TPR;
  const int sl = tid % TPR;  // this thread's slice of the head dim
  const bool row_ok = qi < seq_q;
  const int qlim = qi + offset;  // last visible key (causal)
  const float c = a.qk_scale;    // softmax scale * log2(e); any sign

  float q[DPT], o[DPT];
  {
    const T* qp = (const T*)a.q + (int64_t)b * a.sqb + (int64_t)hq * a.sqh + (qtok0 + (row_ok ? qi : 0)) * a.sqn +
                  sl * DPT;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
      q[e] = row_ok ? to_f32<T>(qp[e]) : 0.f;
      o[e] = 0.f;
    }
  }
  float m_run = NEG_INF, l_run = 0.f;

  const T* kbase = (const T*)a.k + (int64_t)b * a.skb + (int64_t)kvh * a.skh + ktok0 * a.skn;
  const T* vbase = (const T*)a.v + (int64_t)b * a.svb + (int64_t)kvh * a.svh + ktok0 * a.svn;

  for (int n0 = 0; n0 < khi; n0 += BN) {
    // K/V tile -> LDS as fp32; keys past khi are zeros (they are also masked below)
    for (int i = tid; i < BN * (D / 4); i += 256) {
      const int j = i / (D / 4), d4 = (i % (D / 4)) * 4;
      const int n = n0 + j;
      float4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
      if (n < khi) {
        const T* kp = kbase + (int64_t)n * a.skn + d4;
        const T* vp = vbase + (int64_t)n * a.svn + d4;
        kv = float4{to_f32<T>(kp[0]), to_f32<T>(kp[1]), to_f32<T>(kp[2]), to_f32<T>(kp[3])};
        vv = float4{to_f32<T>(vp[0]), to_f32<T>(vp[1]), to_f32<T>(vp[2]), to_f32<T>(vp[3])};
      }
      *(float4*)(ks + j * LDK + d4) = kv;
      *(float4*)(vs + j * LDK + d4) = vv;
    }
    __syncthreads();

    // scores of the tile (log2 domain), excluded keys -inf
    float s[BN];
    float mt = NEG_INF;
#pragma unroll
    for (int j = 0; j < BN; ++j) {
      const float* kr = ks + j * LDK + sl * DPT;
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < DPT; e += 4) {
        const float4 kv = *(const float4*)(kr + e);
        acc = __builtin_fmaf(q[e], kv.x, acc);
        acc = __builtin_fmaf(q[e + 1], kv.y, acc);
        acc = __builtin_fmaf(q[e + 2], kv.z, acc);
        acc = __builtin_fmaf(q[e + 3], kv.w, acc);
      }
      // the four threads of a query are lanes 4r..4r+3: combine their partial sums
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      const int n = n0 + j;
      const bool ok = (n < khi) & ((a.causal == 0) | (n <= qlim));
      s[j] = ok ? acc * c : NEG_INF;
      mt = fmaxf(mt, s[j]);
    }
    const float m_new = fmaxf(m_run, mt);
    const float m_safe = (m_new == NEG_INF) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_safe);  // 0 while m_run is -inf
    l_run *= alpha;
#pragma unroll
    for (int e = 0; e < DPT; ++e) o[e] *= alpha;
    m_run = m_new;
#pragma unroll
    for (int j = 0; j < BN; ++j) {
      const float p = fast_exp2(s[j] - m_safe);
      l_run += p;
      const float* vr = vs + j * LDK + sl * DPT;
#pragma unroll
      for (int e = 0; e < DPT; e += 4) {
        const float4 vv = *(const float4*)(vr + e);
        o[e] = __builtin_fmaf(p, vv.x, o[e]);
        o[e + 1] = __builtin_fmaf(p, vv.y, o[e + 1]);
        o[e + 2] = __builtin_fmaf(p, vv.z, o[e + 2]);
        o[e + 3] = __builtin_fmaf(p, vv.w, o[e + 3]);
      }
    }
    __syncthreads();
  }

  if (!row_ok) return;
  // Rows that saw no key have l == 0 and emit zeros (triton_fwd.py:163-165).
  const float l_safe = (l_run == 0.f) ? 1.f : l_run;
  const float inv = 1.f / l_safe;
  T* op = (T*)a.o + (int64_t)b * a.sob + (int64_t)hq * a.soh + (qtok0 + qi) * a.son + sl * DPT;
#pragma unroll
  for (int e = 0; e < DPT; ++e) op[e] = (T)(o[e] * inv);
  if (a.lse != nullptr && sl == 0) {
    // natural-log LSE (triton_fwd.py:169-172)
    a.lse[(int64_t)b * a.slb + (int64_t)hq * a.slh + (qtok0 + qi)] = (m_run + __log2f(l_safe)) * kLn2;
  }
}

template <class T, int D>
static hipError_t launch_generic(const TileArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((attn_generic_kernel<T, D>), dim3((unsigned)a.total), dim3(256), 0, stream, a);
  return hipGetLastError();
}

fa_status run_fwd_generic(const fa_fwd_params& p, bool varlen, hipStream_t stream, const char** err) {
  TileArgs a = common_args(p);
  a.o = p.o;
  a.sob = p.o_stride_b;
  a.soh = p.o_stride_h;
  a.son = p.o_stride_n;
  a.lse = p.lse;
  a.slb = p.lse_stride_b;
  a.slh = p.lse_stride_h;
  a.varlen = varlen ? 1 : 0;
  if (varlen) {
    a.cu_q = p.cu_seqlens_q;
    a.cu_k = p.cu_seqlens_k;
    a.nq = p.max_seqlen_q;
    a.nk = p.max_seqlen_k;
    a.sqb = a.skb = a.svb = a.sob = a.slb = 0;  // rows are addressed by packed token index
  }
  if (a.nq <= 0 || p.batch <= 0) return FA_OK;
  a.n_rowblk = (a.nq + 63) / 64;
  const int64_t total = (int64_t)p.batch * p.heads_q * a.n_rowblk;
  if (total > INT32_MAX) {
    *err = "grid too large";
    return FA_ERR_UNSUPPORTED;
  }
  a.total = (int32_t)total;
  // run_fwd sends only fp32 at head dim 16 here
  if (p.dtype != FA_DTYPE_F32 || p.head_dim != 16) {
    *err = "the generic kernel serves fp32 at head_dim 16 only";
    return FA_ERR_UNSUPPORTED;
  }
  return hip_status(launch_generic<float, 16>(a, stream), err);
}

}  // namespace fa
