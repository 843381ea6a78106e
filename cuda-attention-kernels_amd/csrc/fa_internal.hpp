// Internal interface between the C ABI (fa_abi.cpp) and the kernel launchers
// (fa_prefill.hip, fa_splitk.hip).  Not part of the public header.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/fused_attn_hip.h"

namespace fa {

// Kernel arguments of the prefill and split-K kernels, passed by value.  Pointers are raw
// device pointers; strides are in elements of the pointed-to type.
struct TileArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;     // prefill: output in the q dtype; split-K: fp32 partials (layout: part_major)
  float* ml;   // split-K: (max, sum) pairs, laid out like the partials
  float* lse;  // prefill: optional natural-log LSE
  const float* k_scale;
  const float* v_scale;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int64_t sqb, sqh, sqn, skb, skh, skn, svb, svh, svn, sob, soh, son;
  int64_t slb, slh;
  int64_t ssb, ssh;
  int32_t hq, hkv, group;
  int32_t nq, nk;  // dense lengths; varlen: maxima
  int32_t n_rowblk;
  int32_t n_split, split_len;
  int32_t ppw, n_chunk;  // split-K: partitions per workgroup, workgroups per (b, kv-head, row block)
  int32_t total;  // workgroups in the grid
  int32_t kv_groups;  // prefill: (batch, kv-head) pairs
  float qk_scale; // softmax scale * log2(e)
  int32_t causal;
  int32_t varlen;
  // paged K/V (split-K decode): k/v are the page pools, skh/skn (svh/svn) strides inside a page
  const int32_t* block_table;
  const int32_t* seqlens_k;
  int64_t sbt;       // block_table row stride
  int64_t spk, spv;  // page strides of the K and V pools
  int32_t page_size, num_pages;
  // key n -> page slot n / page_size as ((uint64_t)n * page_magic) >> page_magic_shift (exact for
  // n < 2^31: page_magic = ceil(2^page_magic_shift / page_size), page_magic_shift = 31 +
  // ceil(log2(page_size)))
  uint32_t page_magic;
  int32_t page_magic_shift;
  // split-K partial layout: 0 = [B, Hq, Nq, S, D] (row-major), 1 = [B, Hkv, S, G*Nq, D]
  // (partition-major: the rows one workgroup writes for one partition are one block)
  int32_t part_major;
  int32_t o16;  // prefill: O base and strides allow 16-byte stores
  int32_t u_heads, u_items;  // dense prefill schedule: q-heads per scheduling unit, and times n_rowblk
};

struct QuantArgs {
  const void* x;
  uint8_t* x8;
  float* scale;
  int64_t sxb, sxh, sxn;
  int32_t h, n, nblk, total;
};

struct CombineArgs {
  const float* opart;  // normalised fp32 partials
  const float* ml;
  void* o;
  int64_t sob, soh, son;
  float* lse;  // optional natural-log LSE [B, Hq, Nq]
  int64_t slb, slh;
  int32_t hq, nq, n_split;
  int32_t group;       // q-heads per kv-head
  int32_t part_major;  // partial layout, as TileArgs::part_major
};

// Number of rows (q-heads x queries) one split-K workgroup covers, and the
// workgroup shape chosen for a given row count G*Nq.
int splitk_waves_for_rows(int rows);

// TileArgs fields that prefill and split-K share (pointers, strides, heads, scale).
TileArgs common_args(const fa_fwd_params& p);

inline fa_status hip_status(hipError_t e, const char** err) {
  if (e == hipSuccess) return FA_OK;
  *err = hipGetErrorString(e);
  return FA_ERR_HIP;
}

// Launchers.  They assume fa_abi.cpp has validated `p`.
fa_status run_fwd(const fa_fwd_params& p, bool varlen, hipStream_t stream, const char** err);
// fp32 at head dim 16 (fa_generic.hip); run_fwd forwards it here.
fa_status run_fwd_generic(const fa_fwd_params& p, bool varlen, hipStream_t stream, const char** err);
// fp32 at head dims 32 to 256 on the fp32 MFMA (fa_prefill_f32.hip); run_fwd forwards those here.
fa_status run_fwd_f32(const fa_fwd_params& p, bool varlen, hipStream_t stream, const char** err);
fa_status run_quantize_fp8(const fa_quant_params& p, hipStream_t stream, const char** err);
// Largest workspace the no-allocation split-K entry point holds (a static device array per GPU).
constexpr size_t kSplitkScratchBytes = size_t{64} << 20;
// This device's address of that array (looked up once per device), for fa_attention_splitk_noalloc.
fa_status splitk_scratch(void** ptr, const char** err);
// kv: paged K/V (nullptr for a dense cache)
fa_status run_splitk(const fa_fwd_params& p, int32_t split_len, void* workspace, hipStream_t stream,
                     const char** err, const fa_paged_kv* kv = nullptr);

}  // namespace fa
