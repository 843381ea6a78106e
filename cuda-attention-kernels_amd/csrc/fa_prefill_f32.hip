// fp32 FlashAttention-2 prefill on the fp32 matrix cores of MI355X (gfx950), D in {32, 64, 128, 256}.
//
// Serves fp32 Q/K/V: the role of the reference's SIMT kernel attn_fwd_kernel
// (csrc/flash_attn.cu:54-187) and of its Triton kernel's fp32 inputs
// (fused_attn/triton_fwd.py:85-172, 210-222), dense and varlen, with the natural-log LSE
// (triton_fwd.py:169-172).  Both products run on v_mfma_f32_32x32x2_f32, so every product
// and sum is an fp32 operation, and P stays fp32.
//
// A workgroup of 4 waves covers 128 queries of one q-head; wave w owns 32 of them.  K and V
// stream through LDS in 32-key fp32 tiles, double-buffered and filled straight from memory.
//
// Operand layout per 32-key block and wave (lane l: j = l % 32, g = l / 32):
//  - S^T = K Q^T over D/2 steps of k = 2.  Step s pairs d = s (lanes g = 0) with d = D/2 + s
//    (lanes g = 1): A = K (lane: key j, that d), B = Q^T (lane: query j, that d).  A lane
//    thus reads four steps of its K row with one 16-byte LDS read and keeps half of its Q row
//    in registers for the whole kernel.
//  - The C fragment gives lane (j, g) query j's scores of keys 8(r/4) + 4g + r%4, r = 0..15.
//  - O^T += V^T P^T over 16 steps of k = 2.  Step r uses, in lane (j, g), the key
//    8(r/4) + 4g + r%4: the one whose probability the lane holds in register r, so P never
//    moves between lanes.  A = V^T, where row i of d block b is d = DB*i + b (DB = D/32
//    blocks), so one LDS read of a V row (32 bytes at D=256 down to 4 at D=32) feeds the
//    step's DB MFMAs.  At D=256 the fp32 accumulators and half a Q row take 256 registers, so
//    that variant runs one wave per SIMD.
//  - K tiles keep 16-byte chunk c of row n at c ^ swz(n), swz(n) = n % 16 (D >= 64) or
//    (n / 2) % 8 (D = 32, whose 128-byte rows put two rows on one bank line): the 16 rows of
//    one read pass hit 16 different bank groups.  A pass over V reads whole rows, so V needs
//    no swizzle (at D=32 the two row halves of a wave share banks: a 2-way conflict on
//    4-byte reads, small beside the 64-cycle MFMAs they feed).
#include <float.h>

#include <type_traits>

#include "fa_device.hpp"
#include "fa_internal.hpp"

namespace fa {

namespace {

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2)))
attn_fwd_f32_kernel(const TileArgs a) {
  constexpr int NW = 4;
  constexpr int BN = 32;                      // keys per tile: one 32-key MFMA block
  constexpr int TILE = BN * D;                // floats per K (or V) tile
  constexpr int QPW = TILE * 4 / 1024 / NW;   // 1-KiB DMA blocks per wave per tile
  constexpr int DB = D / 32;                  // 32-row d blocks of O^T
  constexpr int HS = D / 2;                   // k = 2 steps of S^T
  static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head dim");
  static_assert(TILE * 4 % (1024 * NW) == 0, "direct loads must split evenly over the waves");
  constexpr float NEG_INF = -__builtin_inff();

  // separate arrays so that the compiler can tell a DMA into one buffer from reads of another
  __shared__ __align__(16) float k_buf0[TILE];
  __shared__ __align__(16) float k_buf1[TILE];
  __shared__ __align__(16) float v_buf0[TILE];
  __shared__ __align__(16) float v_buf1[TILE];

  // ---- work item: (batch or sequence, q-head, 128-query block), rank-major ---------------
  // All (batch, q-head) pairs at one rank run together (heaviest causal blocks first), the
  // q-heads of one kv-head side by side; xcd_remap gives each XCD a contiguous range.
  const int nbh = a.total / a.n_rowblk;
  const int logical = xcd_remap((int)blockIdx.x, a.total);
  const int mrev = logical / nbh;
  const int item = logical % nbh;
  const int hq = item % a.hq;
  const int b = item / a.hq;
  const int kvh = hq / a.group;
  const int rb = a.causal ? (a.n_rowblk - 1 - mrev) : mrev;

  int seq_q = a.nq, seq_k = a.nk;
  int64_t qtok0 = 0, ktok0 = 0;
  if (a.varlen) {
    const int qs = __builtin_amdgcn_readfirstlane(a.cu_q[b]);
    const int ks = __builtin_amdgcn_readfirstlane(a.cu_k[b]);
    seq_q = __builtin_amdgcn_readfirstlane(a.cu_q[b + 1]) - qs;
    seq_k = __builtin_amdgcn_readfirstlane(a.cu_k[b + 1]) - ks;
    qtok0 = qs;
    ktok0 = ks;
  }
  const int r0 = rb * NW * 32;
  if (r0 >= seq_q) return;  // uniform over the workgroup (zero-length sequences exit here)
  const int offset = seq_k - seq_q;  // bottom-right causal alignment (reference.py:24-33)
  int khi = seq_k;
  if (a.causal) khi = min(khi, min(r0 + NW * 32, seq_q) + offset);
  const int n_tiles = khi > 0 ? (khi + BN - 1) / BN : 0;

  // ---- lane roles --------------------------------------------------------------------
  const int tid = (int)threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 5, j = lane & 31;
  const int wr0 = r0 + wave * 32;
  const int qi = wr0 + j;
  const bool row_ok = qi < seq_q;
  const bool wave_active = wr0 < seq_q;
  // keys at or beyond mask_from are not visible to every row of this wave
  int mask_from = khi;
  if (a.causal && wave_active) mask_from = min(khi, wr0 + offset + 1);
  // keys below wave_khi are visible to some row of this wave; later tiles only take part in
  // the DMA and the barriers
  const int wave_khi = !wave_active ? 0 : (a.causal ? min(khi, min(wr0 + 32, seq_q) + offset) : khi);
  const int qlim = qi + offset;  // last key this lane's row may see (causal)

  // A negative scale is applied by negating Q (exact); c = |scale| * log2(e) > 0.
  const float c = fmaxf(fabsf(a.qk_scale), kMinScale);
  const uint32_t qsign = a.qk_scale < 0.f ? 0x80000000u : 0u;

  // ---- Q: half of this lane's row, resident (rows past the end read row 0, zeroed) ----
  float qreg[HS];
  {
    const int64_t qrow = qtok0 + (row_ok ? qi : 0);
    const float* qp = (const float*)a.q + (int64_t)b * a.sqb + (int64_t)hq * a.sqh + qrow * a.sqn + g * HS;
    const uint32_t keep = row_ok ? 0xffffffffu : 0u;
#pragma unroll
    for (int i = 0; i < HS / 4; ++i) {
      const u32x4 w = ld16(qp + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[4 * i + e] = __builtin_bit_cast(float, (w[e] ^ qsign) & keep);
    }
  }

  auto swz = [](int n) __attribute__((always_inline)) { return D >= 64 ? n % 16 : (n >> 1) & 7; };

  // ---- K/V tiles: global -> LDS (loads past the tile's last valid key return zeros) -----
  const uint8_t* kbase = (const uint8_t*)a.k + ((int64_t)b * a.skb + (int64_t)kvh * a.skh + ktok0 * a.skn) * 4;
  const uint8_t* vbase = (const uint8_t*)a.v + ((int64_t)b * a.svb + (int64_t)kvh * a.svh + ktok0 * a.svn) * 4;
  const int64_t krow_bytes = a.skn * 4, vrow_bytes = a.svn * 4;
  auto limit = [&](int n0, int64_t row_bytes) __attribute__((always_inline)) {
    const int valid = min(khi - n0, BN);
    return __builtin_amdgcn_readfirstlane(valid > 0 ? (uint32_t)(valid - 1) * (uint32_t)row_bytes + (uint32_t)(D * 4)
                                                    : 0u);
  };
  auto load_tiles = [&](int n0, float* kd, float* vd) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + (int64_t)n0 * krow_bytes, limit(n0, krow_bytes));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + (int64_t)n0 * vrow_bytes, limit(n0, vrow_bytes));
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      const int blk = wave * QPW + i;
      const int byte = blk * 1024 + lane * 16;
      const int r = byte / (D * 4), p = (byte % (D * 4)) / 16;
      lds_dma16<false>(rk, (uint8_t*)kd + blk * 1024, r * (int)krow_bytes + ((p ^ swz(r)) * 16));
      lds_dma16<false>(rv, (uint8_t*)vd + blk * 1024, r * (int)vrow_bytes + p * 16);
    }
  };

  f32x16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
  float m_run = NEG_INF, l_run = 0.f;  // running max (scaled log2 domain), this lane's row-sum share

  // ---- one 32-key tile --------------------------------------------------------------------
  auto tile = [&](const float* Ks, const float* Vs, int n0) __attribute__((always_inline)) {
    // S^T, in two accumulators so that consecutive MFMAs do not depend on each other
    f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
    for (int s4 = 0; s4 < HS / 4; ++s4) {
      const int chunk = (g * (HS / 4) + s4) ^ swz(j);
      const f32x4 kv = __builtin_bit_cast(f32x4, ld16(Ks + j * D + chunk * 4));
      s0 = mfma_f32(kv[0], qreg[4 * s4 + 0], s0);
      s1 = mfma_f32(kv[1], qreg[4 * s4 + 1], s1);
      s0 = mfma_f32(kv[2], qreg[4 * s4 + 2], s0);
      s1 = mfma_f32(kv[3], qreg[4 * s4 + 3], s1);
    }
    f32x16 sc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = s0[r] + s1[r];
    if (n0 + BN > mask_from) {
      __asm__ volatile("");  // keep the rare masking branch out of the common path
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = n0 + 8 * (r >> 2) + 4 * g + (r & 3);
        const bool ok = (n < khi) & ((a.causal == 0) | (n <= qlim));
        sc[r] = ok ? sc[r] : NEG_INF;
      }
    }
    float mx = sc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = vmax(mx, sc[r]);
    const float m_new = vmax(m_run, max_xor32(mx * c));
    const float m_safe = (m_new == NEG_INF) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_safe);
    m_run = m_new;
    float p[16];
    float rs = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = fast_exp2(__builtin_fmaf(sc[r], c, -m_safe));
      rs += p[r];
    }
    l_run = l_run * alpha + rs;
#pragma unroll
    for (int d = 0; d < DB; ++d) oacc[d] *= alpha;
    // O^T += V^T P^T
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float* vp = Vs + (8 * (r >> 2) + 4 * g + (r & 3)) * D + DB * j;
      if constexpr (DB == 8) {
        const f32x4 w0 = __builtin_bit_cast(f32x4, ld16(vp)), w1 = __builtin_bit_cast(f32x4, ld16(vp + 4));
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          oacc[d] = mfma_f32(w0[d], p[r], oacc[d]);
          oacc[d + 4] = mfma_f32(w1[d], p[r], oacc[d + 4]);
        }
      } else if constexpr (DB == 4) {
        const f32x4 w = __builtin_bit_cast(f32x4, ld16(vp));
#pragma unroll
        for (int d = 0; d < 4; ++d) oacc[d] = mfma_f32(w[d], p[r], oacc[d]);
      } else if constexpr (DB == 2) {
        const f32x2 w = __builtin_bit_cast(f32x2, ld8(vp));
#pragma unroll
        for (int d = 0; d < 2; ++d) oacc[d] = mfma_f32(w[d], p[r], oacc[d]);
      } else {
        oacc[0] = mfma_f32(*vp, p[r], oacc[0]);
      }
    }
  };

  // ---- main loop, unrolled by 2 so that every buffer is named at compile time ------------
  if (n_tiles > 0) load_tiles(0, k_buf0, v_buf0);
  auto step = [&](auto stage_tag, int t) __attribute__((always_inline)) {
    constexpr int ST = decltype(stage_tag)::value;
    const float* kc = ST == 0 ? k_buf0 : k_buf1;  // holds tile t
    const float* vc = ST == 0 ? v_buf0 : v_buf1;
    float* kn = ST == 0 ? k_buf1 : k_buf0;  // held tile t-1 (every wave is done with it), takes t+1
    float* vn = ST == 0 ? v_buf1 : v_buf0;
    lds_dma_wait();
    __syncthreads();
    if (t + 1 < n_tiles) load_tiles((t + 1) * BN, kn, vn);
    if (t * BN < wave_khi) tile(kc, vc, t * BN);
  };
  for (int t = 0; t < n_tiles; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < n_tiles) step(std::integral_constant<int, 1>{}, t + 1);
  }

  // ---- epilogue ------------------------------------------------------------------------
  if (!wave_active) return;
  const float l_tot = sum_xor32(l_run);
  if (!row_ok) return;
  // rows that saw no key have l == 0 and emit zeros (triton_fwd.py:163-165)
  const float l_safe = (l_tot == 0.f) ? 1.f : l_tot;
  const float inv = 1.f / l_safe;
  float* op = (float*)a.o + (int64_t)b * a.sob + (int64_t)hq * a.soh + (qtok0 + qi) * a.son;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = 8 * (r >> 2) + 4 * g + (r & 3);  // O^T row of register r: d = DB*i + block
    if constexpr (DB == 1) {
      op[i] = oacc[0][r] * inv;
    } else {
#pragma unroll
      for (int d = 0; d < DB; d += 2) {
        st8(op + DB * i + d, u32x2{__builtin_bit_cast(uint32_t, oacc[d][r] * inv),
                                   __builtin_bit_cast(uint32_t, oacc[d + 1][r] * inv)});
      }
    }
  }
  if (a.lse != nullptr && g == 0) {
    a.lse[(int64_t)b * a.slb + (int64_t)hq * a.slh + (qtok0 + qi)] = (m_run + __log2f(l_safe)) * kLn2;
  }
}

template <int D>
hipError_t launch_f32(const TileArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_f32_kernel<D>), dim3((unsigned)a.total), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

fa_status run_fwd_f32(const fa_fwd_params& p, bool varlen, hipStream_t stream, const char** err) {
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
  a.n_rowblk = (a.nq + 127) / 128;
  const int64_t total = (int64_t)p.batch * p.heads_q * a.n_rowblk;
  if (total > INT32_MAX) {
    *err = "grid too large";
    return FA_ERR_UNSUPPORTED;
  }
  a.total = (int32_t)total;
  const hipError_t e = p.head_dim == 256 ? launch_f32<256>(a, stream)
                       : p.head_dim == 128 ? launch_f32<128>(a, stream)
                       : p.head_dim == 64 ? launch_f32<64>(a, stream)
                                          : launch_f32<32>(a, stream);
  return hip_status(e, err);
}

}  // namespace fa
