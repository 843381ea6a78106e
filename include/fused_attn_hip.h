/*
 * fused_attn_hip.h — C ABI of the MI355X (gfx950) fused-attention backend.
 *
 * This is the drop-in boundary that replaces the reference's pybind module
 * `fused_attn._C` (csrc/bindings.cpp:90-96) and its params struct
 * (csrc/flash_attn.h:9-22), plus the Triton entry points that the reference
 * reached from Python (fused_attn/triton_fwd.py:225-309,
 * fused_attn/triton_splitk.py:140-181, fused_attn/fp8.py:125-147).
 *
 * Conventions
 *  - Plain pointers, element strides and sizes; no framework types.
 *  - All tensor pointers are device pointers on the current HIP device.
 *  - The caller allocates every buffer (outputs and split-K workspace).  The
 *    library never allocates device memory and keeps no pointer after return.
 *  - Every entry point returns an fa_status.  On failure fa_last_error()
 *    returns a thread-local message.  Nothing throws across this boundary and
 *    nothing aborts.
 *  - Work is enqueued on `stream` and is asynchronous, like the reference's
 *    launches on the current CUDA stream (csrc/bindings.cpp:58,78).
 */
#ifndef FUSED_ATTN_HIP_H_
#define FUSED_ATTN_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 6

/* Element types (reference: DType, csrc/flash_attn.h:7). */
typedef enum fa_dtype {
  FA_DTYPE_F16 = 0,
  FA_DTYPE_BF16 = 1,
  FA_DTYPE_F32 = 2,
  FA_DTYPE_FP8_E4M3 = 3 /* OCP float8_e4m3fn, K/V cache only */
} fa_dtype;

typedef enum fa_status {
  FA_OK = 0,
  FA_ERR_INVALID_ARGUMENT = 1, /* shape / stride / alignment / pointer precondition violated */
  FA_ERR_UNSUPPORTED = 2,      /* valid request this backend does not implement (dtype, head_dim) */
  FA_ERR_WORKSPACE = 3,        /* split-K workspace missing or too small */
  FA_ERR_HIP = 4               /* a HIP runtime call or kernel launch failed */
} fa_status;

/*
 * Forward parameters.  Mirrors AttnParams (csrc/flash_attn.h:9-22) with the
 * varlen, LSE and FP8 fields the Triton paths carried as kernel arguments.
 *
 * Dense layout:  q [B, Hq, Nq, D], k/v [B, Hkv, Nk, D], o like q, any strides
 *                with unit stride along D (strides are in elements); k/v token
 *                strides below 16 MiB.
 * Varlen layout: q [total_q, Hq, D], k/v [total_k, Hkv, D]; `batch` is the
 *                number of sequences, cu_seqlens_q/k are device int32 arrays
 *                of batch+1 prefix offsets starting at 0, the *_stride_b
 *                fields are ignored and *_stride_n is the token stride.
 * Head mapping:  q-head h reads kv-head h / (Hq / Hkv) (reference.py:16-21).
 * Causal:        bottom-right aligned, key j visible to query i iff
 *                j <= i + (Nk - Nq) (reference.py:24-33); a row with no
 *                visible key is written as zeros (reference.py:60-61).
 */
typedef struct fa_fwd_params {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t q_stride_b, q_stride_h, q_stride_n;
  int64_t k_stride_b, k_stride_h, k_stride_n;
  int64_t v_stride_b, v_stride_h, v_stride_n;
  int64_t o_stride_b, o_stride_h, o_stride_n;
  int32_t batch, heads_q, heads_kv, seqlen_q, seqlen_k, head_dim;
  float scale;   /* softmax scale; callers pass 1/sqrt(D) for the default (ops.py:89) */
  int32_t causal;
  int32_t dtype;    /* fa_dtype of q and o */
  int32_t kv_dtype; /* fa_dtype of k and v: equal to dtype, or FA_DTYPE_FP8_E4M3 */
  /* varlen (NULL for dense) */
  const int32_t* cu_seqlens_q;
  const int32_t* cu_seqlens_k;
  int32_t max_seqlen_q, max_seqlen_k;
  /* optional natural-log LSE output, fp32 (NULL = not written); reference: WRITE_LSE in
     fused_attn/triton_fwd.py:169-172.  Dense: [B, Hq, Nq] at b*lse_stride_b + h*lse_stride_h + n.
     Varlen: [Hq, total_q] at h*lse_stride_h + token (lse_stride_b unused).  Split-K and paged
     decode write it from the combine, dense layout.  A row without keys gets -inf. */
  float* lse;
  int64_t lse_stride_b, lse_stride_h;
  /* FP8 K/V block scales, fp32 [B, Hkv, ceil(Nk/64)] (fused_attn/fp8.py:31-45);
     used only when kv_dtype == FA_DTYPE_FP8_E4M3 */
  const float* k_scale;
  const float* v_scale;
  int64_t scale_stride_b, scale_stride_h;
} fa_fwd_params;

/* Dense FA2 forward.  Replaces attention_fwd_mma (csrc/bindings.cpp:63-81),
   run_attention_fwd_mma (csrc/flash_attn.h:27), attention_fwd (the SIMT kernel,
   csrc/flash_attn.cu:222-228) and attention_triton (fused_attn/triton_fwd.py:225-265).
   f16/bf16 run on the 16-bit MFMA kernel; f32 on the fp32 MFMA at D in {32, 64, 128, 256} and
   on the generic fp32-math kernel at D = 16.  D in {16, 32, 64, 128, 256}. */
fa_status fa_attention_fwd(const fa_fwd_params* p, void* stream);

/* Packed variable-length forward.  Replaces attention_varlen_triton
   (fused_attn/triton_fwd.py:268-309).  Needs cu_seqlens_q/k and max_seqlen_q; optional LSE. */
fa_status fa_attention_varlen_fwd(const fa_fwd_params* p, void* stream);

/* Bytes of workspace fa_attention_splitk needs for `num_splits` key partitions:
   fp32 partial outputs (B*Hq*Nq*S*D floats), each normalised by its own row sum, plus fp32
   (max, sum) pairs (B*Hq*Nq*S*2 floats) in the log2 domain (the reference keeps fp32
   partials too: fused_attn/triton_splitk.py:90-96,156-158).  The library lays them out as
   [B, Hq, Nq, S, D] or, for 32 or more partitions at D <= 128, as [B, Hkv, S, G*Nq, D]
   (G = Hq/Hkv), so that each workgroup's partials are one contiguous block; the layout is
   internal to the split and combine kernels. */
size_t fa_splitk_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q, int32_t head_dim,
                                 int32_t num_splits);

/* Split-K flash-decoding: one pass per `split_len`-key partition writing normalised fp32
   partials and fp32 log2-domain statistics, then a log-sum-exp combine kernel (which also
   writes the optional LSE).  f16/bf16 q, D in {64, 128, 256}.  Replaces attention_splitk_triton
   (fused_attn/triton_splitk.py:140-181) and, with kv_dtype == FA_DTYPE_FP8_E4M3 and
   k_scale/v_scale set, attention_fp8_triton (fused_attn/fp8.py:125-147).  split_len must be a
   positive multiple of 64; num_splits = ceil(seqlen_k / split_len). */
fa_status fa_attention_splitk(const fa_fwd_params* p, int32_t split_len, void* workspace,
                              size_t workspace_bytes, void* stream);

/* fa_attention_splitk without a caller workspace, for callers that cannot allocate device memory
   (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
   counterpart in the reference.  Same arguments, validation, kernels and results as
   fa_attention_splitk; the workspace is a static device array the library holds on each GPU for
   the life of the process (FA_SPLITK_NOALLOC_MAX_BYTES), so a request whose
   fa_splitk_workspace_bytes exceeds that size fails with FA_ERR_WORKSPACE.  The library calls no
   allocation routine on this path.  Every call on a GPU uses that GPU's one array: calls that
   overlap on one GPU (other streams, other threads) race and must be serialised by the caller.
   No state in the array has to start at zero (each call writes every partial it reads). */
#define FA_SPLITK_NOALLOC_MAX_BYTES ((size_t)64 << 20)
fa_status fa_attention_splitk_noalloc(const fa_fwd_params* p, int32_t split_len, void* stream);

#define FA_MAX_PAGE_SIZE (1 << 24) /* largest page_size fa_attention_paged_decode accepts */

/* Paged (block-table) K/V for fa_attention_paged_decode.  The K and V pools hold
   num_pages pages of page_size keys; p->k / p->v point at the pools and
   p->k_stride_h / k_stride_n (v likewise) are the head and key strides inside a
   page (p->k_stride_b is unused).  Sequence b's key n lives in page
   block_table[b * block_table_stride + n / page_size] at offset n % page_size. */
typedef struct fa_paged_kv {
  const int32_t* block_table;  /* [batch, block_table_cols] page indices, on the device */
  int64_t block_table_stride;  /* elements between rows of block_table */
  int32_t block_table_cols;    /* pages per sequence in the table; cols * page_size >= p->seqlen_k */
  int32_t page_size;           /* keys per page: a positive multiple of 16 (64 for FP8 pools), at most
                                  FA_MAX_PAGE_SIZE */
  const int32_t* seqlens_k;    /* [batch] keys per sequence, on the device; values above p->seqlen_k
                                  are read as p->seqlen_k, negative values as 0 */
  int32_t num_pages;           /* pages per pool; a table entry outside [0, num_pages) reads as zero keys */
  int32_t reserved;
  int64_t k_page_stride, v_page_stride;  /* elements between consecutive pages of each pool */
} fa_paged_kv;

/* Split-K decode over a paged K/V cache: fa_attention_splitk's kernels (same partials,
   combine, workspace size and split_len rules) with each sequence's keys gathered
   through its block table and its own length seqlens_k[b]; p->seqlen_k is the largest
   length (it sizes the grid) and the causal mask is bottom-right per sequence.
   f16/bf16 q, D in {64, 128, 256}.  The reference lists paged K/V for its decode kernels as a
   roadmap item (README.md:224); the semantics are those of attention_splitk_triton
   (fused_attn/triton_splitk.py:140-181) applied to each sequence's gathered keys.
   FP8 pools (p->kv_dtype == FA_DTYPE_FP8_E4M3): the semantics of attention_fp8_triton
   (fused_attn/fp8.py:125-147) on each sequence's gathered keys.  page_size must then be a
   multiple of 64 and p->k_scale / p->v_scale point at fp32 scale pools
   [num_pages, Hkv, page_size / 64] (the 64-key block scales of each page, as
   fused_attn/fp8.py:31-45 computes them for a [num_pages, Hkv, page_size, D] pool), with
   p->scale_stride_b the elements between pages and p->scale_stride_h between heads; the
   blocks of a page are contiguous.  A page outside [0, num_pages) reads as zero keys. */
fa_status fa_attention_paged_decode(const fa_fwd_params* p, const fa_paged_kv* kv, int32_t split_len,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* Reference split heuristic (fused_attn/triton_splitk.py:130-137):
   min(2*num_cus / (batch*heads), seqlen_k / 256, 64), 1 for seqlen_q > 64. */
int32_t fa_choose_num_splits(int32_t batch, int32_t heads, int32_t seqlen_k, int32_t seqlen_q, int32_t num_cus);

/* 1 when `device` is a gfx950 GPU this library has kernels for, else 0.
   Replaces has_tensor_core_kernel (csrc/bindings.cpp:83-86). */
int32_t fa_device_supported(int32_t device);

/* Thread-local description of the last failure on this thread ("" if none). */
const char* fa_last_error(void);

/* FP8 KV-cache quantiser input: x [batch, heads, seqlen, head_dim] in f32/f16/bf16 with element
   strides (unit head_dim stride); outputs x8 contiguous e4m3fn bytes [batch, heads, seqlen, head_dim]
   and fp32 scales [batch, heads, ceil(seqlen/64)]. */
typedef struct fa_quant_params {
  const void* x;
  int64_t x_stride_b, x_stride_h, x_stride_n;
  int32_t batch, heads, seqlen, head_dim;
  int32_t dtype; /* fa_dtype of x: F16, BF16 or F32 */
  void* x8;
  float* scale;
} fa_quant_params;

/* Per-(batch, head, 64-key block) absmax/448 scaling and e4m3fn rounding, bit-identical to the
   reference's torch chain quantize_kv_fp8 (fused_attn/fp8.py:31-45).  head_dim in {16, 32, 64, 128, 256}. */
fa_status fa_quantize_kv_fp8(const fa_quant_params* p, void* stream);

/* FA_ABI_VERSION of the loaded library. */
int32_t fa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FUSED_ATTN_HIP_H_ */
