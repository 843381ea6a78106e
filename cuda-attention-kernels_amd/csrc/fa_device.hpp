// Device helpers for the gfx950 (CDNA4) attention kernels: vector types, MFMA
// wrappers, fp8 decode, LDS transpose reads and cross-lane reductions.
//
// Lane layouts (wave64) used throughout, verified on MI355X:
//   v_mfma_f32_32x32x16_{bf16,f16}:  A[i][k]: lane l holds i = l%32, k = 8*(l/32) + 0..7
//                                    B[k][j]: lane l holds j = l%32, k = 8*(l/32) + 0..7
//                                    C[i][j]: lane l, acc r holds i = 8*(r/4) + 4*(l/32) + r%4, j = l%32
//   v_mfma_f32_16x16x32_{bf16,f16}:  A[i][k]: lane l holds i = l%16, k-group l/16 (8 values)
//                                    B[k][j]: lane l holds j = l%16, k-group l/16 (8 values)
//                                    C[i][j]: lane l, acc r holds i = 4*(l/16) + r, j = l%16
//   ds_read_b64_tr_b16: in each 16-lane group, lane i receives element (i%4) of the
//                       8-byte rows addressed by lanes (i/4) + 4e, e = 0..3.
//   v_permlane32_swap(x, x): {r0, r1} with max(r0, r1) = max(x[l], x[l^32]).
//   ds_read_b64_tr_b8:  in each 16-lane group, lane i receives byte (i%8) of the
//                       8-byte rows addressed by lanes (i%16)/8 + 2e, e = 0..7.
//   v_cvt_pk_f32_fp8: OCP float8_e4m3fn -> fp32, exact for all 256 codes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fa {

typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef _Float16 f16x8 __attribute__((__vector_size__(16)));
typedef __bf16 bf16x2 __attribute__((__vector_size__(4)));
typedef _Float16 f16x2 __attribute__((__vector_size__(4)));
typedef float f32x16 __attribute__((__vector_size__(64)));
typedef float f32x4 __attribute__((__vector_size__(16)));
typedef float f32x2 __attribute__((__vector_size__(8)));
typedef short i16x4 __attribute__((__vector_size__(8)));
typedef int i32x2 __attribute__((__vector_size__(8)));
typedef uint32_t u32x4 __attribute__((__vector_size__(16)));
typedef uint32_t u32x2 __attribute__((__vector_size__(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element tags.  Storage is always 16-bit (or 8-bit for fp8) in memory.
struct BF16 {
  static constexpr int bytes = 2;
};
struct F16 {
  static constexpr int bytes = 2;
};
struct FP8 {  // OCP float8_e4m3fn K/V cache
  static constexpr int bytes = 1;
};

template <class E>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c);

template <>
__device__ __forceinline__ f32x16 mfma32<BF16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<F16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

template <class E>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c);
template <>
__device__ __forceinline__ f32x4 mfma16<BF16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<F16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

// A operand of a 16x16x32 MFMA that turns a 32x32x16 B fragment into row sums.
// A 32x32x16 B fragment (K = 16 keys, N = 32 rows) puts row l % 32, keys 8 * (l / 32) + i in
// lane l.  Read as the B operand of a 16x16x32 MFMA, lane l is column l % 16 and k-group
// l / 16, so column n gathers row n (groups 0 and 2) and row n + 16 (groups 1 and 3).  With
// A[m][k] = 1 exactly when the k-group's parity equals that of m / 4, output rows m with even
// m / 4 sum row n and the others row n + 16; in the 16x16 output layout (lane l holds rows
// 4 * (l / 16) .. + 3 of column l % 16) every lane then holds the full 16-key sum of its own
// row l % 32, in all four registers.
template <class E>
__device__ __forceinline__ u32x4 rowsum_ones(int lane) {
  const uint32_t one2 = std::is_same<E, BF16>::value ? 0x3f803f80u : 0x3c003c00u;
  const uint32_t w = (((lane >> 4) ^ (lane >> 2)) & 1) ? 0u : one2;
  return u32x4{w, w, w, w};
}

// Round-to-nearest-even pack of two fp32 into one dword of 16-bit values (lo first).
template <class E>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  f16x2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// 16-bit -> fp32 (exact).
template <class E>
__device__ __forceinline__ float lo_f32(uint32_t w);
template <class E>
__device__ __forceinline__ float hi_f32(uint32_t w);
template <>
__device__ __forceinline__ float lo_f32<BF16>(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
template <>
__device__ __forceinline__ float hi_f32<BF16>(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
template <>
__device__ __forceinline__ float lo_f32<F16>(uint32_t w) {
  return (float)__builtin_bit_cast(f16x2, w)[0];
}
template <>
__device__ __forceinline__ float hi_f32<F16>(uint32_t w) {
  return (float)__builtin_bit_cast(f16x2, w)[1];
}

// Four e4m3fn bytes (one dword) -> two dwords of packed 16-bit E values.  Exact:
// every e4m3fn value is representable in bf16 and in fp16.
template <class E>
__device__ __forceinline__ u32x2 fp8x4_to_e(uint32_t w) {
  const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  u32x2 r;
  r[0] = pack2<E>(a[0], a[1]);
  r[1] = pack2<E>(b[0], b[1]);
  return r;
}

// acc + lo + hi of a dword holding two 16-bit values, via v_dot2 with (1, 1):
// the exact sum of the rounded values, one instruction per pair.
template <class E>
__device__ __forceinline__ float sum2(uint32_t w, float acc);
template <>
__device__ __forceinline__ float sum2<BF16>(uint32_t w, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
}
template <>
__device__ __forceinline__ float sum2<F16>(uint32_t w, float acc) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
}

// Raw buffer resource over [base, base + num_bytes): loads at offsets >= num_bytes
// return zeros (hardware range check), which zero-fills tails without branches.
// Callers pass wave-uniform values; the readfirstlanes state that to the compiler, so
// the descriptor always lives in SGPRs (a descriptor it cannot prove uniform is used
// through a per-lane "waterfall" loop around every load: measured 16x slower).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)addr);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(lo | (hi << 32)), (short)0,
                                           (int)__builtin_amdgcn_readfirstlane(num_bytes), 0x00020000);
}
// 16-byte buffer load; STREAM sets the non-temporal hint for data read exactly once.
template <bool STREAM>
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, int offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, STREAM ? 2 : 0);
}

// 16-byte buffer load written straight into LDS (no VGPRs): lane l's 16 bytes land at
// lds + 16*l; `lds` must be wave-uniform.  Completion is tracked by vmcnt.
template <bool STREAM>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void* lds, int offset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, offset, 0, 0,
                                           STREAM ? 2 : 0);
#else
  (void)r, (void)lds, (void)offset;
#endif
}
// Wait until every outstanding vector-memory load of this wave (including LDS DMA) landed.
__device__ __forceinline__ void lds_dma_wait() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt unconstrained (gfx9 encoding)
}

// Online-softmax rescale threshold (log2 units): the running max is only
// raised, and O rescaled, once a row's max grows by more than this.
constexpr float kRescaleLog2 = 8.0f;

// Smallest score multiplier the kernels use: a masked score (-inf) times it stays -inf.
constexpr float kMinScale = 1e-30f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Maximum of scores as v_maximum3_f32 (IEEE 754-2019 maximum: NaN-propagating, like
// torch.max).  fmaxf (maxNum) would first canonicalise every MFMA result with an extra
// v_max_f32 x, x, x: one more VALU instruction per score.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return vmax(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// 8-byte transposed LDS read (ds_read_b64_tr_b16).  `p` points into __shared__ memory.
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef i16x4 __attribute__((address_space(3))) * lds_v4_ptr;
  typedef uint16_t __attribute__((address_space(3))) * lds_u16_ptr;
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4_ptr)((lds_u16_ptr)p));
  return __builtin_bit_cast(u32x2, r);
#else
  (void)p;
  return u32x2{0, 0};
#endif
}

// 8-byte transposed LDS read of 8-bit elements (ds_read_b64_tr_b8).  Within each
// group of 16 lanes, lane i receives byte i % 8 of the 8-byte pieces addressed by
// lanes (i % 16) / 8 + 2e of its group, e = 0..7, in order of e.
__device__ __forceinline__ u32x2 lds_read_tr8(const uint8_t* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef i32x2 __attribute__((address_space(3))) * lds_v2_ptr;
  typedef uint8_t __attribute__((address_space(3))) * lds_u8_ptr;
  const i32x2 r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2_ptr)((lds_u8_ptr)p));
  return __builtin_bit_cast(u32x2, r);
#else
  (void)p;
  return u32x2{0, 0};
#endif
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, const u32x2& v) { *reinterpret_cast<u32x2*>(p) = v; }

// Physical workgroup id -> logical id such that each XCD (8 per MI355X, each
// with its own L2) receives a contiguous range of logical ids.  Workgroups are
// dispatched round-robin over XCDs, so id p runs on XCD p % 8.
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  constexpr int kXcds = 8;
  const int q = total / kXcds, r = total % kXcds;
  const int xcd = pid % kXcds, slot = pid / kXcds;
  return xcd * q + (xcd < r ? xcd : r) + slot;
}

}  // namespace fa
