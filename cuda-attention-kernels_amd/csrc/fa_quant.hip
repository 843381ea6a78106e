// FP8 (OCP e4m3fn) KV-cache quantiser: the write side of the FP8 decode path.
//
// Same arithmetic, in the same order, as the reference's torch chain
// quantize_kv_fp8 (fused_attn/fp8.py:31-45), so the bytes and scales are equal to
// torch's on the same inputs:
//   scale = max(amax|x_block|, 1e-12) / 448      per (batch, kv-head, 64-key block)
//   x8    = e4m3fn(clamp(x / scale, -448, 448))   round to nearest even
// with torch's NaN propagation (a NaN in a block makes its amax, scale and bytes NaN).
// Padding keys past N are zeros, as the reference's F.pad, so they do not change amax.
//
// One wave per 64-key block; the bytes are converted in pairs (v_cvt_pk_fp8_f32) and
// stored 16 at a time.  Reads 2 (or 4) bytes and writes 1 byte per element: HBM-bound.
#include <math.h>

#include "fa_device.hpp"
#include "fa_internal.hpp"

namespace fa {

namespace {

constexpr int kQBlock = 64;
constexpr float kE4M3Max = 448.0f;

// amax / 448 as torch evaluates a tensor divided by a Python scalar on the GPU: a
// multiply by the fp32 reciprocal 1/448 (rounded once, on the host)
__device__ __forceinline__ float block_scale(float amax) { return amax * (1.0f / kE4M3Max); }

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// element e of a 16-element chunk held as raw 32-bit words, widened to fp32 (exact)
template <class T>
__device__ __forceinline__ float chunk_elem(const uint32_t* w, int e) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(w[e]);
  } else if constexpr (__is_same(T, __bf16)) {
    return __uint_as_float((e & 1) ? (w[e / 2] & 0xffff0000u) : (w[e / 2] << 16));
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? (w[e / 2] >> 16) : (w[e / 2] & 0xffffu)));
  }
}

// e4m3fn byte pair of values already clamped to [-448, 448] or NaN: round to nearest
// even by the hardware conversion; NaN is S.1111.111 with the value's sign, as torch writes it
__device__ __forceinline__ uint32_t e4m3_pair(float s0, float s1) {
  uint32_t pk = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s0, s1, 0, false) & 0xffffu;
  if (s0 != s0) pk = (pk & 0xff00u) | 0x7fu | ((__float_as_uint(s0) >> 24) & 0x80u);
  if (s1 != s1) pk = (pk & 0x00ffu) | 0x7f00u | ((__float_as_uint(s1) >> 16) & 0x8000u);
  return pk;
}

// x / scale, correctly rounded, for finite x and a finite positive scale with y = RN(1/scale):
// one product and one FMA residual correction (Markstein's theorem: y within half an ulp of
// 1/scale and a faithful first quotient give the correctly rounded quotient; checked bit for
// bit against the IEEE division over every fp32 x with x / scale in [2^-12, 449] for 64
// scales, the range in which the quotient can reach a nonzero e4m3 code).  The sign is x's,
// which also gives -0 for x = -0.
__device__ __forceinline__ float div_by_scale(float x, float scale, float y) {
  const float q0 = x * y;
  const float r = __builtin_fmaf(-q0, scale, x);
  return __builtin_copysignf(__builtin_fmaf(r, y, q0), x);
}

// elements per lane-chunk: one 16-byte load, so every load instruction of a wave reads 1 KB
// of consecutive input (measured: fp32 chunks of 16 elements, four loads at a 64-byte lane
// stride, ran at 0.54 of HBM bandwidth against 0.74 for 16-byte chunks)
template <class T>
constexpr int kQuantChunk = 16 / (int)sizeof(T);

// waves per 64-key block for key rows of ROW_BYTES
template <int ROW_BYTES>
constexpr int kQuantWaves = ROW_BYTES > 256 ? ROW_BYTES / 256 : 1;

// WPB waves per 64-key block, so that a wave holds at most 16 KB of input (one wave for
// 16-bit D <= 128 and fp32 D <= 64, two or four above).  Lanes hold chunks of CH consecutive
// elements of one key row (16 bytes of input): step j of wave w takes chunk
// (j * WPB + w) * 64 + lane of the block's [64][D] elements, so each load instruction reads
// 1 KB of consecutive input and each store writes CH bytes per lane.  The block's amax is a
// wave reduction (plus an LDS exchange between the waves of a block).  Loads and stores are
// non-temporal: the input is read once and the output is not re-read.
template <class T, int D, int CH>
__global__ void __launch_bounds__(64 * kQuantWaves<D * (int)sizeof(T)>) quantize_kv_fp8_kernel(const QuantArgs a) {
  constexpr int WPB = kQuantWaves<D * (int)sizeof(T)>;
  constexpr int STEPS = D / (CH * WPB);            // chunks per lane: 64 * D / (WPB * 64 lanes * CH)
  constexpr int CW = CH * (int)sizeof(T) / 4;      // 32-bit words per chunk
  static_assert(D % CH == 0 && STEPS >= 1 && CW % 4 == 0 && CH % 4 == 0, "a chunk stays inside one key row");

  const int blk = (int)blockIdx.x % a.nblk;
  const int bh = (int)blockIdx.x / a.nblk;
  const int h = bh % a.h;
  const int b = bh / a.h;
  const int lane = (int)threadIdx.x & 63;
  const int wave = (int)threadIdx.x >> 6;
  const T* x = (const T*)a.x + (int64_t)b * a.sxb + (int64_t)h * a.sxh;
  // the block's bytes are one contiguous run of the [B, H, N, D] output
  uint8_t* x8 = a.x8 + (((int64_t)b * a.h + h) * a.n + (int64_t)blk * kQBlock) * D;
  const int nkeys = min(kQBlock, a.n - blk * kQBlock);

  uint32_t raw[STEPS][CW];
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    const int i = ((j * WPB + wave) * 64 + lane) * CH;
    const int key = i / D, d = i % D;
    if (key < nkeys) {
      const u32x4* src = (const u32x4*)(x + (int64_t)(blk * kQBlock + key) * a.sxn + d);
#pragma unroll
      for (int c = 0; c < CW / 4; ++c) {
        const u32x4 t = __builtin_nontemporal_load(src + c);
        raw[j][4 * c] = t.x, raw[j][4 * c + 1] = t.y, raw[j][4 * c + 2] = t.z, raw[j][4 * c + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int c = 0; c < CW; ++c) raw[j][c] = 0u;  // the zero padding of the last block
    }
  }
  // amax over |x| as integers: for non-negative floats the integer order is the float order
  // and every NaN sorts above +inf, so the maximum propagates NaN as torch.amax does
  uint32_t amax_bits = 0;
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
#pragma unroll
    for (int e = 0; e < CH; ++e) amax_bits = max(amax_bits, __float_as_uint(chunk_elem<T>(raw[j], e)) & 0x7fffffffu);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax_bits = max(amax_bits, (uint32_t)__shfl_xor((int)amax_bits, off));
  if constexpr (WPB > 1) {
    __shared__ uint32_t red[WPB];
    if (lane == 0) red[wave] = amax_bits;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < WPB; ++w) amax_bits = max(amax_bits, red[w]);
  }
  const bool finite = amax_bits < 0x7f800000u;  // uniform over the workgroup
  float amax = __uint_as_float(amax_bits);
  if (finite) amax = fmaxf(amax, 1e-12f);  // clamp_min; inf and NaN pass through
  const float scale = block_scale(amax);
  if (threadIdx.x == 0) a.scale[(int64_t)bh * a.nblk + blk] = scale;
  const float y = __fdiv_rn(1.0f, scale);

#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    uint32_t w[CH / 4];
    if (finite) {
      // every x is finite and |x / scale| <= 448 * (1 + 2^-22): no NaN can arise
#pragma unroll
      for (int t = 0; t < CH / 4; ++t) {
        float s[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          s[u] = fminf(fmaxf(div_by_scale(chunk_elem<T>(raw[j], 4 * t + u), scale, y), -kE4M3Max), kE4M3Max);
        w[t] = ((uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s[0], s[1], 0, false) & 0xffffu) |
               ((uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(s[2], s[3], 0, false) << 16);
      }
    } else {
      // a block holding inf or NaN: the IEEE division (inf / inf and x / NaN make NaN) and
      // NaN-preserving clamps
#pragma unroll
      for (int t = 0; t < CH / 4; ++t) {
        float s[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          s[u] = __fdiv_rn(chunk_elem<T>(raw[j], 4 * t + u), scale);
          if (s[u] == s[u]) s[u] = fminf(fmaxf(s[u], -kE4M3Max), kE4M3Max);
        }
        w[t] = e4m3_pair(s[0], s[1]) | (e4m3_pair(s[2], s[3]) << 16);
      }
    }
    const int i = ((j * WPB + wave) * 64 + lane) * CH;
    if (i / D < nkeys) {
      if constexpr (CH == 16) {
        __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, (u32x4*)(x8 + i));
      } else if constexpr (CH == 8) {
        __builtin_nontemporal_store(u32x2{w[0], w[1]}, (u32x2*)(x8 + i));
      } else {
        __builtin_nontemporal_store(w[0], (uint32_t*)(x8 + i));
      }
    }
  }
}

template <class T, int D>
hipError_t launch_quant(const QuantArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((quantize_kv_fp8_kernel<T, D, kQuantChunk<T>>), dim3((unsigned)a.total), dim3(64 * kQuantWaves<D * (int)sizeof(T)>), 0,
                     stream, a);
  return hipGetLastError();
}

template <class T>
hipError_t launch_quant_d(const QuantArgs& a, int d, hipStream_t stream) {
  switch (d) {
    case 16:
      return launch_quant<T, 16>(a, stream);
    case 32:
      return launch_quant<T, 32>(a, stream);
    case 64:
      return launch_quant<T, 64>(a, stream);
    case 128:
      return launch_quant<T, 128>(a, stream);
    case 256:
      return launch_quant<T, 256>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

fa_status run_quantize_fp8(const fa_quant_params& p, hipStream_t stream, const char** err) {
  QuantArgs a{};
  a.x = p.x;
  a.x8 = (uint8_t*)p.x8;
  a.scale = p.scale;
  a.sxb = p.x_stride_b;
  a.sxh = p.x_stride_h;
  a.sxn = p.x_stride_n;
  a.h = p.heads;
  a.n = p.seqlen;
  a.nblk = (p.seqlen + kQBlock - 1) / kQBlock;
  const int64_t total = (int64_t)p.batch * p.heads * a.nblk;
  if (total == 0) return FA_OK;
  if (total > INT32_MAX) {
    *err = "grid too large";
    return FA_ERR_UNSUPPORTED;
  }
  a.total = (int32_t)total;
  hipError_t e = hipErrorInvalidValue;
  switch (p.dtype) {
    case FA_DTYPE_F32:
      e = launch_quant_d<float>(a, p.head_dim, stream);
      break;
    case FA_DTYPE_BF16:
      e = launch_quant_d<__bf16>(a, p.head_dim, stream);
      break;
    case FA_DTYPE_F16:
      e = launch_quant_d<_Float16>(a, p.head_dim, stream);
      break;
    default:
      break;
  }
  return hip_status(e, err);
}

}  // namespace fa
