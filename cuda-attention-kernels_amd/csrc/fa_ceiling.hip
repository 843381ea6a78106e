// Matrix-core ceiling probe for the 16-bit prefill kernel (a measurement aid, built into its own
// library, libfa_probe.so; not part of the attention ABI).
//
// Every wave streams independent v_mfma_f32_32x32x16_bf16 (four accumulator chains) on register
// operands loaded once from random bf16 data, eight waves per CU (two per SIMD, one workgroup per
// CU, as the 8-wave prefill kernel runs), with no LDS, memory or vector work in the loop.  The
// rate it reaches is what the matrix cores sustain on the board under MFMA load, clock and power
// management included, which the spec peak (2.4 GHz) does not say.  bench.py reports it beside
// the prefill workload.
#include <hip/hip_runtime.h>

#include "fa_device.hpp"

namespace fa {

// Floats of LDS each workgroup reserves: 96 KiB, so one workgroup (eight waves) runs per CU.
constexpr int kCeilingLdsFloats = 24576;
// Random bf16 elements the operands are read from (the host passes at least this many).
constexpr int kCeilingDataElems = 64 * 4096 + 4096;

__global__ void __launch_bounds__(512) mfma_ceiling_kernel(const uint16_t* data, float* out, int iters) {
  __shared__ float hold[kCeilingLdsFloats];
  const int tid = (int)threadIdx.x, lane = tid & 63;
  // operands differ per lane and per workgroup block: offsets stay below kCeilingDataElems
  const uint16_t* p = data + (size_t)(blockIdx.x % 64) * 4096 + lane * 8;
  u32x4 a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = ld16(p + j * 512);
    b[j] = ld16(p + 2048 + j * 512);
  }
  f32x16 acc[4] = {};
#pragma unroll 4
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = mfma32<BF16>(a[j], b[j], acc[j]);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  }
  hold[tid] = s;
  __syncthreads();
  out[(size_t)blockIdx.x * 512 + tid] = hold[511 - tid];
}

}  // namespace fa

// Launches `grid` workgroups of 512 threads, each wave running `iters` rounds of four MFMAs;
// `data` holds at least fa_probe_data_elems() bf16 values and `out` grid * 512 floats.
// 0 on success, else the HIP error code.
extern "C" int fa_probe_data_elems() { return fa::kCeilingDataElems; }

extern "C" int fa_probe_mfma_ceiling(const void* data, float* out, int grid, int iters, void* stream) {
  if (data == nullptr || out == nullptr || grid <= 0 || iters <= 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(fa::mfma_ceiling_kernel, dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream,
                     (const uint16_t*)data, out, iters);
  return (int)hipGetLastError();
}
