// extern "C" entry points of libfused_attn_hip.so: argument validation, error
// reporting, device checks.  Replaces the reference's pybind layer
// (csrc/bindings.cpp:10-96): the checks mirror check_inputs
// (csrc/bindings.cpp:35-50) and the mma preconditions (:66-74), but failures
// are returned as fa_status codes with a thread-local message instead of
// exceptions, and the caller owns every allocation.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/fused_attn_hip.h"
#include "fa_internal.hpp"

static_assert(FA_SPLITK_NOALLOC_MAX_BYTES == fa::kSplitkScratchBytes, "header limit and scratch array size differ");

namespace {

thread_local std::string g_last_error;

fa_status fail(fa_status code, const char* msg) {
  g_last_error = msg;
  return code;
}

bool aligned(const void* p, size_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

size_t dtype_bytes(int32_t dt) {
  switch (dt) {
    case FA_DTYPE_F16:
    case FA_DTYPE_BF16:
      return 2;
    case FA_DTYPE_F32:
      return 4;
    case FA_DTYPE_FP8_E4M3:
      return 1;
    default:
      return 0;
  }
}

// Validation shared by every forward entry point.  `fp8_ok` allows FP8 K/V (split-K);
// `generic_ok` also allows fp32 and head dims 16 and 32 (prefill and varlen, where the MFMA kernel
// takes 16-bit D in {16, 32, 64, 128, 256} and fp32 runs on the fp32 MFMA kernel or the generic one).
fa_status validate(const fa_fwd_params* p, bool varlen, bool fp8_ok, bool generic_ok) {
  if (p == nullptr) return fail(FA_ERR_INVALID_ARGUMENT, "params is NULL");
  if (p->batch < 0 || p->heads_q <= 0 || p->heads_kv <= 0 || p->seqlen_q < 0 || p->seqlen_k < 0 ||
      p->head_dim <= 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "sizes must be non-negative (heads and head_dim positive)");
  if (p->heads_q % p->heads_kv != 0) return fail(FA_ERR_INVALID_ARGUMENT, "H_q must be a multiple of H_kv");
  if (dtype_bytes(p->dtype) == 0 || dtype_bytes(p->kv_dtype) == 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "unknown dtype code");
  if (p->dtype != FA_DTYPE_F16 && p->dtype != FA_DTYPE_BF16 && !(generic_ok && p->dtype == FA_DTYPE_F32))
    return fail(FA_ERR_UNSUPPORTED, generic_ok ? "q/o dtype must be float16, bfloat16 or float32"
                                               : "q/o dtype must be float16 or bfloat16 for split-K");
  if (p->kv_dtype != p->dtype) {
    if (!(fp8_ok && p->kv_dtype == FA_DTYPE_FP8_E4M3))
      return fail(FA_ERR_INVALID_ARGUMENT, "k/v dtype must match q (or be float8_e4m3fn on the split-K path)");
  }
  const int d = p->head_dim;
  if (generic_ok ? !(d == 16 || d == 32 || d == 64 || d == 128 || d == 256) : !(d == 64 || d == 128 || d == 256))
    return fail(FA_ERR_UNSUPPORTED, generic_ok ? "head_dim must be 16, 32, 64, 128 or 256"
                                               : "head_dim must be 64, 128 or 256 on the split-K path");
  if (p->kv_dtype == FA_DTYPE_FP8_E4M3 && (p->k_scale == nullptr || p->v_scale == nullptr))
    return fail(FA_ERR_INVALID_ARGUMENT, "FP8 K/V needs k_scale and v_scale");
  if (!(p->scale == p->scale)) return fail(FA_ERR_INVALID_ARGUMENT, "scale is NaN");

  if (varlen) {
    if (p->cu_seqlens_q == nullptr || p->cu_seqlens_k == nullptr)
      return fail(FA_ERR_INVALID_ARGUMENT, "varlen needs cu_seqlens_q and cu_seqlens_k");
    if (p->max_seqlen_q < 0 || p->max_seqlen_k < 0)
      return fail(FA_ERR_INVALID_ARGUMENT, "max_seqlen must be non-negative");
  }
  const bool empty = p->batch == 0 || (varlen ? p->max_seqlen_q == 0 : p->seqlen_q == 0);
  if (empty) return FA_OK;

  const bool no_keys = varlen ? p->max_seqlen_k == 0 : p->seqlen_k == 0;
  if (p->q == nullptr || p->o == nullptr || (!no_keys && (p->k == nullptr || p->v == nullptr)))
    return fail(FA_ERR_INVALID_ARGUMENT, "q, k, v and o must be non-NULL");
  // 16-byte vector loads of Q rows and K/V rows; 8-byte stores of O.
  const int64_t qvec = 16 / dtype_bytes(p->dtype), kvvec = (int64_t)(16 / dtype_bytes(p->kv_dtype)),
                ovec = 8 / dtype_bytes(p->dtype);
  if (!aligned(p->q, 16) || !aligned(p->k, 16) || !aligned(p->v, 16) || !aligned(p->o, 8))
    return fail(FA_ERR_INVALID_ARGUMENT, "q/k/v must be 16-byte aligned and o 8-byte aligned");
  if ((!varlen && (p->q_stride_b % qvec)) || p->q_stride_h % qvec || p->q_stride_n % qvec)
    return fail(FA_ERR_INVALID_ARGUMENT, "q strides must be multiples of 16 bytes");
  if ((!varlen && (p->k_stride_b % kvvec || p->v_stride_b % kvvec)) || p->k_stride_h % kvvec ||
      p->k_stride_n % kvvec || p->v_stride_h % kvvec || p->v_stride_n % kvvec)
    return fail(FA_ERR_INVALID_ARGUMENT, "k/v strides must be multiples of 16 bytes");
  if ((!varlen && (p->o_stride_b % ovec)) || p->o_stride_h % ovec || p->o_stride_n % ovec)
    return fail(FA_ERR_INVALID_ARGUMENT, "o strides must be multiples of 8 bytes");
  // K/V tiles are addressed with signed 32-bit byte offsets of up to 128 rows (the prefill
  // kernel's tiles at D <= 64) from the tile start: 127 rows of a stride below 16 MiB stay
  // below 2^31
  const int64_t kvb = (int64_t)dtype_bytes(p->kv_dtype);
  if (p->k_stride_n < 0 || p->v_stride_n < 0 || p->k_stride_n * kvb >= (1 << 24) || p->v_stride_n * kvb >= (1 << 24))
    return fail(FA_ERR_UNSUPPORTED, "k/v token stride must be below 16 MiB");
  return FA_OK;
}

}  // namespace

extern "C" {

fa_status fa_attention_fwd(const fa_fwd_params* p, void* stream) {
  g_last_error.clear();
  fa_status st = validate(p, /*varlen=*/false, /*fp8_ok=*/false, /*generic_ok=*/true);
  if (st != FA_OK) return st;
  if (p->lse != nullptr && (p->lse_stride_b < 0 || p->lse_stride_h < 0))
    return fail(FA_ERR_INVALID_ARGUMENT, "negative LSE stride");
  const char* err = nullptr;
  st = fa::run_fwd(*p, false, reinterpret_cast<hipStream_t>(stream), &err);
  if (st != FA_OK) return fail(st, err ? err : "launch failed");
  return FA_OK;
}

fa_status fa_attention_varlen_fwd(const fa_fwd_params* p, void* stream) {
  g_last_error.clear();
  fa_status st = validate(p, /*varlen=*/true, /*fp8_ok=*/false, /*generic_ok=*/true);
  if (st != FA_OK) return st;
  if (p->lse != nullptr && p->lse_stride_h < 0) return fail(FA_ERR_INVALID_ARGUMENT, "negative LSE stride");
  const char* err = nullptr;
  st = fa::run_fwd(*p, true, reinterpret_cast<hipStream_t>(stream), &err);
  if (st != FA_OK) return fail(st, err ? err : "launch failed");
  return FA_OK;
}

size_t fa_splitk_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q, int32_t head_dim,
                                 int32_t num_splits) {
  if (batch <= 0 || heads_q <= 0 || seqlen_q <= 0 || head_dim <= 0 || num_splits <= 0) return 0;
  const size_t rows = (size_t)batch * (size_t)heads_q * (size_t)seqlen_q * (size_t)num_splits;
  // fp32 normalised partial outputs, then fp32 (max, sum) pairs
  return rows * ((size_t)head_dim * sizeof(float) + 2 * sizeof(float));
}

fa_status fa_attention_splitk(const fa_fwd_params* p, int32_t split_len, void* workspace, size_t workspace_bytes,
                              void* stream) {
  g_last_error.clear();
  fa_status st = validate(p, /*varlen=*/false, /*fp8_ok=*/true, /*generic_ok=*/false);
  if (st != FA_OK) return st;
  if (p->lse != nullptr && (p->lse_stride_b < 0 || p->lse_stride_h < 0))
    return fail(FA_ERR_INVALID_ARGUMENT, "negative LSE stride");
  if (split_len <= 0 || split_len % 64 != 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "split_len must be a positive multiple of 64");
  if (p->batch == 0 || p->seqlen_q == 0) return FA_OK;
  const int32_t splits = p->seqlen_k > 0 ? (p->seqlen_k + split_len - 1) / split_len : 1;
  const size_t need = fa_splitk_workspace_bytes(p->batch, p->heads_q, p->seqlen_q, p->head_dim, splits);
  if (workspace == nullptr || workspace_bytes < need) {
    char buf[160];
    snprintf(buf, sizeof(buf), "split-K workspace too small: need %zu bytes, got %zu", need,
             workspace == nullptr ? (size_t)0 : workspace_bytes);
    return fail(FA_ERR_WORKSPACE, buf);
  }
  if (!aligned(workspace, 16)) return fail(FA_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  if (p->kv_dtype == FA_DTYPE_FP8_E4M3 && (p->scale_stride_b < 0 || p->scale_stride_h < 0))
    return fail(FA_ERR_INVALID_ARGUMENT, "negative FP8 scale stride");
  const char* err = nullptr;
  st = fa::run_splitk(*p, split_len, workspace, reinterpret_cast<hipStream_t>(stream), &err);
  if (st != FA_OK) return fail(st, err ? err : "launch failed");
  return FA_OK;
}

fa_status fa_attention_splitk_noalloc(const fa_fwd_params* p, int32_t split_len, void* stream) {
  g_last_error.clear();
  fa_status st = validate(p, /*varlen=*/false, /*fp8_ok=*/true, /*generic_ok=*/false);
  if (st != FA_OK) return st;
  if (p->lse != nullptr && (p->lse_stride_b < 0 || p->lse_stride_h < 0))
    return fail(FA_ERR_INVALID_ARGUMENT, "negative LSE stride");
  if (split_len <= 0 || split_len % 64 != 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "split_len must be a positive multiple of 64");
  if (p->batch == 0 || p->seqlen_q == 0) return FA_OK;
  if (p->kv_dtype == FA_DTYPE_FP8_E4M3 && (p->scale_stride_b < 0 || p->scale_stride_h < 0))
    return fail(FA_ERR_INVALID_ARGUMENT, "negative FP8 scale stride");
  const int32_t splits = p->seqlen_k > 0 ? (p->seqlen_k + split_len - 1) / split_len : 1;
  const size_t need = fa_splitk_workspace_bytes(p->batch, p->heads_q, p->seqlen_q, p->head_dim, splits);
  if (need > fa::kSplitkScratchBytes) {
    char buf[200];
    snprintf(buf, sizeof(buf),
             "split-K needs %zu bytes of workspace here; the no-allocation entry point holds at most %zu "
             "(use longer partitions, or fa_attention_splitk with a caller workspace)",
             need, fa::kSplitkScratchBytes);
    return fail(FA_ERR_WORKSPACE, buf);
  }
  const char* err = nullptr;
  void* scratch = nullptr;
  st = fa::splitk_scratch(&scratch, &err);
  if (st != FA_OK) return fail(st, err ? err : "scratch lookup failed");
  st = fa::run_splitk(*p, split_len, scratch, reinterpret_cast<hipStream_t>(stream), &err);
  if (st != FA_OK) return fail(st, err ? err : "launch failed");
  return FA_OK;
}

fa_status fa_attention_paged_decode(const fa_fwd_params* p, const fa_paged_kv* kv, int32_t split_len,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (p == nullptr || kv == nullptr) return fail(FA_ERR_INVALID_ARGUMENT, "params is NULL");
  fa_fwd_params q = *p;
  q.k_stride_b = q.v_stride_b = 0;  // keys are found through the block table
  fa_status st = validate(&q, /*varlen=*/false, /*fp8_ok=*/true, /*generic_ok=*/false);
  if (st != FA_OK) return st;
  if (q.lse != nullptr && (q.lse_stride_b < 0 || q.lse_stride_h < 0))
    return fail(FA_ERR_INVALID_ARGUMENT, "negative LSE stride");
  if (split_len <= 0 || split_len % 64 != 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "split_len must be a positive multiple of 64");
  if (kv->page_size <= 0 || kv->page_size % 16 != 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "page_size must be a positive multiple of 16");
  if (kv->page_size > FA_MAX_PAGE_SIZE)
    return fail(FA_ERR_INVALID_ARGUMENT, "page_size must be at most 2^24 keys");
  const bool fp8 = q.kv_dtype == FA_DTYPE_FP8_E4M3;
  if (fp8 && kv->page_size % 64 != 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "FP8 pools need page_size a multiple of 64 (64-key scale blocks)");
  if (fp8 && (q.scale_stride_b < 0 || q.scale_stride_h < 0))
    return fail(FA_ERR_INVALID_ARGUMENT, "negative FP8 scale stride");
  if (kv->num_pages < 0 || kv->block_table_cols < 0) return fail(FA_ERR_INVALID_ARGUMENT, "negative page count");
  if (q.batch == 0 || q.seqlen_q == 0) return FA_OK;
  if (kv->block_table == nullptr || kv->seqlens_k == nullptr)
    return fail(FA_ERR_INVALID_ARGUMENT, "block_table and seqlens_k must be non-NULL");
  if (!aligned(kv->block_table, 4) || !aligned(kv->seqlens_k, 4))
    return fail(FA_ERR_INVALID_ARGUMENT, "block_table and seqlens_k must be 4-byte aligned");
  if (q.batch > 1 && kv->block_table_stride < kv->block_table_cols)
    return fail(FA_ERR_INVALID_ARGUMENT, "block_table rows overlap (stride below cols)");
  if ((int64_t)kv->block_table_cols * kv->page_size < q.seqlen_k)
    return fail(FA_ERR_INVALID_ARGUMENT, "block_table has fewer pages per sequence than seqlen_k needs");
  const int64_t kvvec = 16 / (int64_t)dtype_bytes(q.kv_dtype);
  if (kv->k_page_stride < 0 || kv->v_page_stride < 0 || kv->k_page_stride % kvvec || kv->v_page_stride % kvvec)
    return fail(FA_ERR_INVALID_ARGUMENT, "page strides must be non-negative multiples of 16 bytes");
  const int32_t splits = q.seqlen_k > 0 ? (q.seqlen_k + split_len - 1) / split_len : 1;
  const size_t need = fa_splitk_workspace_bytes(q.batch, q.heads_q, q.seqlen_q, q.head_dim, splits);
  if (workspace == nullptr || workspace_bytes < need) {
    char buf[160];
    snprintf(buf, sizeof(buf), "split-K workspace too small: need %zu bytes, got %zu", need,
             workspace == nullptr ? (size_t)0 : workspace_bytes);
    return fail(FA_ERR_WORKSPACE, buf);
  }
  if (!aligned(workspace, 16)) return fail(FA_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  const char* err = nullptr;
  st = fa::run_splitk(q, split_len, workspace, reinterpret_cast<hipStream_t>(stream), &err, kv);
  if (st != FA_OK) return fail(st, err ? err : "launch failed");
  return FA_OK;
}

int32_t fa_choose_num_splits(int32_t batch, int32_t heads, int32_t seqlen_k, int32_t seqlen_q, int32_t num_cus) {
  if (seqlen_q > 64) return 1;  // prefill-sized queries already fill the GPU
  const int64_t programs = (int64_t)batch * heads;
  int64_t want = (2 * (int64_t)num_cus) / (programs > 1 ? programs : 1);
  if (want < 1) want = 1;
  int64_t cap = seqlen_k / 256;
  if (cap < 1) cap = 1;
  int64_t n = want < cap ? want : cap;
  return (int32_t)(n < 64 ? n : 64);
}

int32_t fa_device_supported(int32_t device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

const char* fa_last_error(void) { return g_last_error.c_str(); }

fa_status fa_quantize_kv_fp8(const fa_quant_params* p, void* stream) {
  g_last_error.clear();
  if (p == nullptr) return fail(FA_ERR_INVALID_ARGUMENT, "params is NULL");
  if (p->batch < 0 || p->heads < 0 || p->seqlen < 0) return fail(FA_ERR_INVALID_ARGUMENT, "sizes must be non-negative");
  const int d = p->head_dim;
  if (!(d == 16 || d == 32 || d == 64 || d == 128 || d == 256))
    return fail(FA_ERR_UNSUPPORTED, "head_dim must be 16, 32, 64, 128 or 256");
  if (p->dtype != FA_DTYPE_F32 && p->dtype != FA_DTYPE_F16 && p->dtype != FA_DTYPE_BF16)
    return fail(FA_ERR_UNSUPPORTED, "x must be float32, float16 or bfloat16");
  if (p->batch == 0 || p->heads == 0 || p->seqlen == 0) return FA_OK;
  if (p->x == nullptr || p->x8 == nullptr || p->scale == nullptr)
    return fail(FA_ERR_INVALID_ARGUMENT, "x, x8 and scale must be non-NULL");
  if (p->x_stride_b < 0 || p->x_stride_h < 0 || p->x_stride_n < 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "negative stride");
  // the kernel reads x in 16-byte vectors along head_dim and stores x8 in 8-byte words
  const int64_t vec = 16 / (int64_t)dtype_bytes(p->dtype);
  if (p->x_stride_b % vec || p->x_stride_h % vec || p->x_stride_n % vec)
    return fail(FA_ERR_INVALID_ARGUMENT, "x strides must be multiples of 16 bytes");
  if (!aligned(p->x, 16) || !aligned(p->x8, 16) || !aligned(p->scale, 4))
    return fail(FA_ERR_INVALID_ARGUMENT, "x and x8 must be 16-byte aligned, scale 4-byte aligned");
  const char* err = nullptr;
  const fa_status st = fa::run_quantize_fp8(*p, reinterpret_cast<hipStream_t>(stream), &err);
  if (st != FA_OK) return fail(st, err ? err : "launch failed");
  return FA_OK;
}

int32_t fa_abi_version(void) { return FA_ABI_VERSION; }

}  // extern "C"
