// Split-K flash-decoding kernels for MI355X (gfx950).
//
//   * attn_splitk_kernel: the reference's _attn_splitk_kernel
//     (fused_attn/triton_splitk.py:29-96), including the FP8 K/V variant of
//     _attn_fp8_kernel (fused_attn/fp8.py:59-122): one partial output per key
//     partition plus its (max, sum) statistics in the log2 domain.  Partials are fp32,
//     as the reference keeps them (triton_splitk.py:90-96,156-158), so the combine adds
//     no rounding beyond fp32; each is stored normalised by its own sum (a convex
//     combination of V rows, O_s / l_s), which the combine weighs by l_s;
//   * splitk_combine_kernel: the log-sum-exp merge of the partitions
//     (_splitk_combine_kernel, fused_attn/triton_splitk.py:99-127).
//
// Work decomposition.  Keys are cut into partitions of split_len keys (the unit the
// partials and the combine work on).  A workgroup streams `ppw` consecutive
// partitions of one (batch, kv-head) through LDS and writes one partial per
// partition, so the fixed cost of a workgroup (Q fragments, the first tile's memory
// latency) is paid once per ppw partitions and the global->LDS pipeline runs across
// partition boundaries without a drain.
//
// A workgroup has NW waves; wave w owns 32 "rows", a row being a (q-head of the kv
// group, query) pair, so the G = Hq/Hkv heads that share a kv-head read each K/V
// tile once.  Per tile, per wave (S^T orientation, so the softmax is lane-local):
//   S^T = K Q^T   v_mfma_f32_32x32x16: A = K rows from LDS, B = Q from VGPRs.
//                 The C fragment gives each lane one row and 16 keys; the A-row ->
//                 key map (kperm) hands each lane 8 contiguous keys per 16-key step.
//   softmax       online, base 2, scale*log2(e) folded in; max/sum need only the
//                 partner lane l^32 (v_permlane32_swap).
//   P^T           rounded to 16 bits in place: the B operand of the next MFMA.
//   O^T += V^T P^T  A = V^T read from row-major LDS with ds_read_b64_tr_b16.
// K/V go global -> LDS by DMA (buffer_load ... lds) in their storage type; FP8 K/V
// stay 8-bit in LDS (half the LDS per stage, so more workgroups per CU) and are
// widened to 16 bits when read as MFMA operands, V through ds_read_b64_tr_b8.
// LDS holds two stages (tile t+1 loads while tile t is read), or, for one-wave
// workgroups where LDS rather than registers bounds the workgroups per CU, a single
// stage whose K and V halves are refilled as soon as they have been read (the choice
// is made per launch in launch_split_nw).
//
// Paged K/V (PAGED): each sequence's keys live in pages of a shared pool, found
// through its block-table row, and each sequence has its own length.  A workgroup
// loads the block-table entries of its key range once (lane i holds entry i, up to
// 256 entries in four VGPRs); each 32-key half of a tile lies inside one page (page
// sizes are multiples of 32), so its buffer descriptor is built from one entry read
// with v_readlane, and the DMA addressing inside the tile is unchanged.  An entry
// outside [0, num_pages) gets an empty descriptor: its keys read as zeros.  FP8 pools carry
// their block scales per page, [num_pages, Hkv, page_size / 64] (page sizes are then
// multiples of 64, so a 64-key scale block lies inside one page); a page outside the pool
// gets scale 0, so its keys stay zero keys.
#include <float.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "fa_device.hpp"
#include "fa_internal.hpp"
#include "fa_tile.hpp"

namespace fa {

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits 3:0 and 15:14), other counters unconstrained.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// s_waitcnt lgkmcnt(0), other counters unconstrained.
__device__ __forceinline__ void lgkm_wait0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Workgroup barrier without a memory fence (__syncthreads adds one, which waits for every
// outstanding load, LDS DMA included).  LDS written by DMA is published by each wave's own
// vmcnt wait before the barrier; LDS reads are retired by lgkm_wait0 before it.  One-wave
// workgroups need no barrier, only the compiler ordering.
template <int NW>
__device__ __forceinline__ void wg_barrier() {
  if constexpr (NW > 1) {
    __asm__ volatile("s_barrier" ::: "memory");
  } else {
    __asm__ volatile("" ::: "memory");
  }
}

template <int D, class E, class KV, int NW, int BN, bool PAGED, bool ONE_STAGE, int PGS>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2)))
attn_splitk_kernel(const TileArgs a) {
  using Shape = TileShape<D, BN>;    // 16-bit tiles
  using Shape8 = TileShape8<D, BN>;  // FP8 tiles
  constexpr bool IS_FP8 = KV::bytes == 1;
  constexpr int TILE_BYTES = BN * D * KV::bytes;  // one K (or V) tile
  constexpr int KB = BN / 32;   // 32-key MFMA blocks per tile
  constexpr int KS = D / 16;    // k-steps of S^T = K Q^T
  constexpr int DB = D / 32;    // 32-wide d blocks of O^T
  // one DMA wave instruction fills 1 KiB = 64 lanes x 16 B
  constexpr int QPW = (TILE_BYTES / 1024) / NW;
  static_assert(BN % 32 == 0 && D % 32 == 0 && (D == 64 || D == 128 || D == 256), "tile shape");
  static_assert(TILE_BYTES % (1024 * NW) == 0, "tile loads must split evenly over the waves");
  constexpr int PG_REGS = 4;  // paged: block-table entries held per lane (64 * PG_REGS per workgroup)
  // paged: keys per page group, the unit one buffer descriptor covers (32, or 16 for pages of
  // 16 + 32k keys); a 1-KiB DMA block holds 2-8 whole rows, so it never straddles a group
  constexpr int NPG = BN / PGS;
  static_assert(PGS == 16 || PGS == 32, "page group");
  constexpr float NEG_INF = -__builtin_inff();

  // Two LDS stages (tile t+1 loads while tile t is read), or, for one-wave workgroups, a
  // single stage: K and V in arrays of their own, each refilled as soon as it has been
  // read.  That halves the LDS of a workgroup, so more fit on a CU; it pays where LDS
  // rather than registers bounds the occupancy (chosen at launch).  Every buffer is an
  // array of its own and every access names it at compile time, so the compiler can tell
  // that a DMA filling one buffer never aliases reads of another (and does not wait for
  // that DMA before reading).
  static_assert(!ONE_STAGE || NW == 1, "single stage is for one-wave workgroups");
  constexpr int STAGES = ONE_STAGE ? 1 : 2;
  __shared__ __align__(16) uint8_t lds_st0[STAGES == 2 ? 2 * TILE_BYTES : 16];
  __shared__ __align__(16) uint8_t lds_st1[STAGES == 2 ? 2 * TILE_BYTES : 16];
  __shared__ __align__(16) uint8_t lds_k1[STAGES == 1 ? TILE_BYTES : 16];
  __shared__ __align__(16) uint8_t lds_v1[STAGES == 1 ? TILE_BYTES : 16];

  // ---- work item: (batch, kv-head, chunk of ppw partitions, row block) -------------
  const int logical = xcd_remap((int)blockIdx.x, a.total);
  const int rb = logical % a.n_rowblk;
  int item = logical / a.n_rowblk;
  int chunk, kvh, b;
  if constexpr (PAGED) {
    // kv-head innermost: neighbouring workgroups read the same block-table entries (one
    // row per sequence), which then hit in the scalar cache (measured: paged decode with
    // 128-key partitions 5% faster than with the partition innermost)
    kvh = item % a.hkv;
    item /= a.hkv;
    chunk = item % a.n_chunk;
    b = item / a.n_chunk;
  } else {
    chunk = item % a.n_chunk;
    item /= a.n_chunk;
    kvh = item % a.hkv;
    b = item / a.hkv;
  }

  const int seq_q = a.nq;
  int seq_k = a.nk;
  // paged: this sequence's own length, clamped to the grid's [0, max length]
  if constexpr (PAGED) seq_k = min(max(__builtin_amdgcn_readfirstlane(a.seqlens_k[b]), 0), a.nk);
  const int R = a.group * seq_q;  // rows: (q-head in group, query)
  const int r0 = rb * NW * 32;    // < R: the grid has ceil(R / (NW * 32)) row blocks
  const int offset = seq_k - seq_q;  // bottom-right causal alignment (reference.py:24-33)

  const int part0 = chunk * a.ppw;
  const int part_end = min(part0 + a.ppw, a.n_split);
  const int klo = part0 * a.split_len;
  int khi = min(seq_k, part_end * a.split_len);
  if (a.causal) {
    // last query of the block (rows wrap around the queries once per q-head)
    const int re = min(r0 + NW * 32, R);
    const int qmax = (re - r0 >= seq_q || (r0 % seq_q) > ((re - 1) % seq_q)) ? seq_q - 1 : (re - 1) % seq_q;
    khi = min(khi, qmax + offset + 1);
  }
  const int n_tiles = khi > klo ? (khi - klo + BN - 1) / BN : 0;
  const int tiles_per_part = a.split_len / BN;  // split_len is a multiple of 64 (C ABI)

  // ---- lane roles ------------------------------------------------------------------
  const int tid = (int)threadIdx.x;
  // wave index is uniform per wave: keep it (and every per-wave bound) in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 5, j = lane & 31;
  const int wr0 = r0 + wave * 32;
  const int row = wr0 + j;
  const bool row_ok = row < R;
  const bool wave_active = wr0 < R;
  const int hq = kvh * a.group + (row_ok ? row / seq_q : 0);
  const int qi = row_ok ? row % seq_q : 0;
  // Keys visible to every row of the wave need no element-wise mask; keys at or
  // beyond wave_khi are visible to no row of the wave.
  int wave_khi = khi, mask_from = khi;
  if (a.causal && wave_active) {
    const int we = min(wr0 + 32, R);
    int qlo, qhi;
    if (we - wr0 >= seq_q || (wr0 % seq_q) > ((we - 1) % seq_q)) {
      qlo = 0;
      qhi = seq_q - 1;
    } else {
      qlo = wr0 % seq_q;
      qhi = (we - 1) % seq_q;
    }
    wave_khi = min(khi, qhi + offset + 1);
    mask_from = min(khi, qlo + offset + 1);
  }

  // K/V of this (batch, kv-head), read with buffer loads: a load past the
  // resource's byte limit returns zeros, which zero-fills the keys >= khi of the
  // last tile without branches (masked keys must not carry NaN/Inf into P*V).
  // (paged: the pools' base for this kv-head; the batch strides are 0)
  const uint8_t* kbase = (const uint8_t*)a.k + ((int64_t)b * a.skb + (int64_t)kvh * a.skh) * KV::bytes;
  const uint8_t* vbase = (const uint8_t*)a.v + ((int64_t)b * a.svb + (int64_t)kvh * a.svh) * KV::bytes;
  const int64_t krow_bytes = a.skn * KV::bytes, vrow_bytes = a.svn * KV::bytes;
  const float* ksc = nullptr;
  const float* vsc = nullptr;
  // FP8: the accumulator holds O / v_cur, v_cur being the V block scale of a recent tile, and
  // v_cur goes back in, in fp32, when a partial is emitted.  A tile whose V block scale vb lies
  // within a factor 2 of v_cur folds vb / v_cur (in [1/2, 2]) into P before P's 16-bit rounding;
  // any other tile first re-expresses the accumulator in its own scale (O *= v_cur / vb, fp32),
  // so P is never scaled by more than 2 either way.  The reference multiplies each block's
  // P*V by v_scale after the product, in fp32 (fp8.py:116); folding v_scale itself into P would
  // push P * v_scale (v_scale = amax / 448) into fp16's subnormal range for V of small
  // magnitude, and folding a ratio to a workgroup-wide maximum scale would do the same for
  // small-V blocks that sit beside a large-V block.
  float v_cur = IS_FP8 ? 0.f : 1.f;
  if (KV::bytes == 1) {
    // (paged: the scale pools' base for this kv-head; a block's scale is at page * ssb + its
    // 64-key block inside the page)
    ksc = a.k_scale + (PAGED ? 0 : (int64_t)b * a.ssb) + (int64_t)kvh * a.ssh;
    vsc = a.v_scale + (PAGED ? 0 : (int64_t)b * a.ssb) + (int64_t)kvh * a.ssh;
  }

  // A negative softmax scale is applied by negating Q (exact for 16-bit floats),
  // so the kernel always works with c = |scale| * log2(e) > 0 and max(c*s) = c*max(s).
  // c is kept away from 0 so that a masked score (-inf) times c stays -inf; for a
  // zero scale every 2^(c*s) is then 1 to float precision, as for c = 0.
  const uint32_t qsign = a.qk_scale < 0.f ? 0x80008000u : 0u;
  const float c_abs = fmaxf(fabsf(a.qk_scale), kMinScale);

  // ---- paged: the block-table entries of keys [klo, khi) --------------------------
  int pg[PG_REGS] = {};
  int first_slot = 0;
  int first_pages[NPG];  // the first tile's pages: uniform loads through the scalar cache,
                        // which the K/V stream does not evict, so the first DMA waits little
  if constexpr (PAGED) {
    // bounded by the grid's largest length, not this sequence's, so that this load does
    // not wait for seqlens_k[b] (both are in flight together); <= block_table_cols.
    // Issued before the Q loads: waiting for the entries then leaves Q in flight.
    first_slot = klo / a.page_size;
    const int kgrid = min(a.nk, part_end * a.split_len);
    const int slot_end = kgrid > klo ? (kgrid - 1) / a.page_size + 1 : first_slot;
    const int32_t* bt = a.block_table + (int64_t)b * a.sbt;
#pragma unroll
    for (int h = 0; h < NPG; ++h) {
      const int nh = klo + PGS * h;
      first_pages[h] = nh < kgrid ? bt[nh / a.page_size] : -1;
    }
#pragma unroll
    for (int r = 0; r < PG_REGS; ++r) {
      const int sl = first_slot + 64 * r + (tid & 63);
      pg[r] = sl < slot_end ? bt[sl] : -1;
    }
  }
  // ---- Q fragments (B operand of S^T), resident for the whole kernel -------------
  // (rows past the end read row 0 of the item, which exists, and are then zeroed:
  // the loads stay unconditional and are all in flight together)
  u32x4 qf[KS];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (int64_t)b * a.sqb + (int64_t)hq * a.sqh + (int64_t)qi * a.sqn + 8 * g;
    const uint32_t keep = row_ok ? 0xffffffffu : 0u;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = (ld16(qp + 16 * s) ^ qsign) & keep;
  }
  // keep the Q loads ahead of the first K/V tiles' DMA: waiting for Q then leaves the tiles in flight
  __builtin_amdgcn_sched_barrier(0);

  // page slot of key n >= 0: a multiply-high in place of a division by the page size
  auto slot_of = [&](int n) __attribute__((always_inline)) {
    return (int)(((uint64_t)(uint32_t)n * a.page_magic) >> a.page_magic_shift);
  };
  // page of key n (paged; n in [klo, khi), so its slot is among the loaded entries)
  auto page_of = [&](int n) __attribute__((always_inline)) {
    const int rel = __builtin_amdgcn_readfirstlane(slot_of(n) - first_slot);
    const int ln = rel & 63;
    int v = __builtin_amdgcn_readlane(pg[0], ln);
    if (rel >= 64) v = __builtin_amdgcn_readlane(pg[1], ln);
    if (rel >= 128) v = __builtin_amdgcn_readlane(pg[2], ln);
    if (rel >= 192) v = __builtin_amdgcn_readlane(pg[3], ln);
    return v;
  };
  // paged: descriptors of the PGS-key groups of the tile starting at n0; keys at or past
  // khi, and pages outside the pool, are beyond the byte limit and read as zeros
  auto paged_resources = [&](int n0, __amdgpu_buffer_rsrc_t* rk, __amdgpu_buffer_rsrc_t* rv) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < NPG; ++h) {
      const int nh = n0 + PGS * h;
      const int valid = min(khi - nh, PGS);
      const int page = valid <= 0 ? -1 : (n0 == klo ? first_pages[h] : page_of(nh));
      const bool ok = valid > 0 && (uint32_t)page < (uint32_t)a.num_pages;
      const int64_t off = ok ? (int64_t)(nh - slot_of(nh) * a.page_size) : 0;
      const int64_t pgk = ok ? (int64_t)page * a.spk : 0, pgv = ok ? (int64_t)page * a.spv : 0;
      const uint32_t klim = __builtin_amdgcn_readfirstlane(
          ok ? (uint32_t)(valid - 1) * (uint32_t)krow_bytes + (uint32_t)(D * KV::bytes) : 0u);
      const uint32_t vlim = __builtin_amdgcn_readfirstlane(
          ok ? (uint32_t)(valid - 1) * (uint32_t)vrow_bytes + (uint32_t)(D * KV::bytes) : 0u);
      rk[h] = make_rsrc(kbase + pgk * KV::bytes + off * krow_bytes, klim);
      rv[h] = make_rsrc(vbase + pgv * KV::bytes + off * vrow_bytes, vlim);
    }
  };

  // ---- K/V tiles: global -> LDS (K rows permuted by kperm) ---------------------------
  auto resources = [&](int n0, __amdgpu_buffer_rsrc_t& rk, __amdgpu_buffer_rsrc_t& rv) __attribute__((always_inline)) {
    // Byte limit = end of the tile's last key below khi.  It fits 32 bits (BN * row
    // bytes < 2^31, checked at the C ABI) and is wave-uniform, so the descriptor lives
    // in SGPRs.  Valid for any row stride, including 0 for a single-key cache.
    const int valid = min(khi - n0, BN);
    const uint32_t klim = __builtin_amdgcn_readfirstlane(
        valid > 0 ? (uint32_t)(valid - 1) * (uint32_t)krow_bytes + (uint32_t)(D * KV::bytes) : 0u);
    const uint32_t vlim = __builtin_amdgcn_readfirstlane(
        valid > 0 ? (uint32_t)(valid - 1) * (uint32_t)vrow_bytes + (uint32_t)(D * KV::bytes) : 0u);
    rk = make_rsrc(kbase + (int64_t)n0 * krow_bytes, klim);
    rv = make_rsrc(vbase + (int64_t)n0 * vrow_bytes, vlim);
  };
  // Each wave fills QPW 1-KiB blocks of the K and of the V tile straight from memory.
  auto load_parts = [&](int n0, uint8_t* kl, uint8_t* vl, bool do_k, bool do_v) __attribute__((always_inline)) {
    if constexpr (PAGED) {
      __amdgpu_buffer_rsrc_t rk[NPG], rv[NPG];
      paged_resources(n0, rk, rv);
#pragma unroll
      for (int i = 0; i < QPW; ++i) {
        const int blk = wave * QPW + i;
        const int byte = blk * 1024 + lane * 16;
        const int r = byte / (D * KV::bytes), p = (byte % (D * KV::bytes)) / 16;
        // a 1-KiB block holds 2-8 whole rows of one page group (kperm only swaps key bits 2
        // and 3, so it keeps a row in its 16-key group)
        const int grp = (blk * 1024 / (D * KV::bytes)) / PGS;  // wave-uniform
        __amdgpu_buffer_rsrc_t ck = rk[0], cv = rv[0];
#pragma unroll
        for (int h = 1; h < NPG; ++h) {
          if (grp == h) {
            ck = rk[h];
            cv = rv[h];
          }
        }
        const int sk = IS_FP8 ? Shape8::swz_k(r) : Shape::swz_k(r);
        const int sv = IS_FP8 ? Shape8::swz_v(r) : Shape::swz_v(r);
        if (do_k) lds_dma16<true>(ck, kl + blk * 1024, (kperm(r) - PGS * grp) * (int)krow_bytes + ((p ^ sk) * 16));
        if (do_v) lds_dma16<true>(cv, vl + blk * 1024, (r - PGS * grp) * (int)vrow_bytes + ((p ^ sv) * 16));
      }
      return;
    }
    __amdgpu_buffer_rsrc_t rk, rv;
    resources(n0, rk, rv);
#pragma unroll
    for (int i = 0; i < QPW; ++i) {
      const int blk = wave * QPW + i;
      const int byte = blk * 1024 + lane * 16;
      const int r = byte / (D * KV::bytes), p = (byte % (D * KV::bytes)) / 16;
      const int sk = IS_FP8 ? Shape8::swz_k(r) : Shape::swz_k(r);
      const int sv = IS_FP8 ? Shape8::swz_v(r) : Shape::swz_v(r);
      if (do_k) lds_dma16<true>(rk, kl + blk * 1024, kperm(r) * (int)krow_bytes + ((p ^ sk) * 16));
      if (do_v) lds_dma16<true>(rv, vl + blk * 1024, r * (int)vrow_bytes + ((p ^ sv) * 16));
    }
  };
  auto load_tile = [&](int n0, uint8_t* stage) __attribute__((always_inline)) {
    load_parts(n0, stage, stage + TILE_BYTES, true, true);
  };
  f32x16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
  // Running max m_run (log2 domain, scaled) and this lane's share of the row sum,
  // both for the current partition.
  float m_run = NEG_INF, l_run = 0.f;

  // Per-lane LDS element offsets (within a stage) of the MFMA operand reads.
  // K: S^T A-operand, row kb*32 + j, logical chunk 2s + g.
  int koffs[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) koffs[s] = j * D + (((2 * s + g) ^ Shape::swz_k(j)) * 8);
  // V: ds_read_b64_tr_b16 sources, rows 8g + 4*hi + (i >> 2) of each 16-key step,
  // columns 32d + 16dh + 4(i & 3); the row term kb*32 + 16h is a constant offset.
  const int tr_i = lane & 15, tr_dh = (lane >> 4) & 1;
  int voffs[DB][2];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int vr_row = 8 * g + 4 * hi + (tr_i >> 2);
      const int col = 32 * d + 16 * tr_dh + 4 * (tr_i & 3);
      voffs[d][hi] = vr_row * D + (((col >> 3) ^ Shape::swz_v(vr_row)) * 8) + (col & 7);
    }
  }
  // FP8 tiles (byte offsets).  K: A-operand row j, 8 bytes at d = 16s + 8g.
  int koffs8[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) koffs8[s] = j * D + ((s ^ Shape8::swz_k(j)) * 16) + 8 * g;
  // V: ds_read_b64_tr_b8 sources.  Lane p of 16-lane group G points at row
  // 8(G/2) + (p%16)/2 of the 16-key step, bytes 32d + 16(G%2) + 8(p%2), so that lane l
  // receives keys 8(l/32) + 0..7 of d = 32d + l%32: the A layout of O^T += V^T P^T.
  int voffs8[DB];
  {
    const int grp = lane >> 4, r8 = 8 * (grp >> 1) + ((lane & 15) >> 1);
#pragma unroll
    for (int d = 0; d < DB; ++d) voffs8[d] = r8 * D + (((2 * d + (grp & 1)) ^ Shape8::swz_v(r8)) * 16) + 8 * (lane & 1);
  }
  const int qlim = qi + offset;  // last key this lane's row may see (causal)

  // Partial of partition `part` in fp32, normalised by its row sum, plus its log2-domain
  // statistics (triton_splitk.py:90-96); then the state restarts for the next partition.
  // A partition with no visible key (l = 0) stores zeros.
  auto emit_partial = [&](int part, uint8_t* stage = nullptr) __attribute__((always_inline)) {
    const float l_tot = sum_xor32(l_run);  // each lane summed its 16 of the row's keys per tile
    const float inv = l_tot > 0.f ? v_cur / l_tot : 0.f;
    const int vr = min(32, R - wr0);  // rows of this wave
    // partition-major: this wave's rows of the partition are vr consecutive rows
    const int64_t prow0 = ((int64_t)(b * a.hkv + kvh) * a.n_split + part) * R + wr0;
    if (NW == 1 && a.part_major && stage != nullptr && wave_active && vr * D * 4 <= 2 * TILE_BYTES) {
      // Staged through the LDS stage the last tile was read from: the wave's rows go out as
      // one contiguous block with every lane storing 16 bytes, instead of 16 stores per lane
      // from the vr * 2 lanes that hold them (measured on the FP8 decode cache with 128-key
      // partitions: +2.8%).  One wave: its LDS accesses run in order, no barrier needed.
      float* sp = (float*)stage;
      if (row_ok) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const int d0 = d * 32 + 8 * rq + 4 * g;  // this lane's 4 consecutive elements
            *(f32x4*)(sp + j * D + d0) = f32x4{oacc[d][4 * rq] * inv, oacc[d][4 * rq + 1] * inv,
                                               oacc[d][4 * rq + 2] * inv, oacc[d][4 * rq + 3] * inv};
          }
        }
      }
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      float* op0 = (float*)a.o + prow0 * D;
      const int n16 = vr * D / 4;
      for (int c = lane; c < n16; c += 64) st16(op0 + 4 * c, ld16(sp + 4 * c));
      if (row_ok && g == 0) st8(a.ml + (prow0 + j) * 2, __builtin_bit_cast(u32x2, f32x2{m_run, l_tot}));
    } else if (wave_active && row_ok) {
      const int64_t prow = a.part_major ? prow0 + j : ((int64_t)(b * a.hq + hq) * seq_q + qi) * a.n_split + part;
      float* op = (float*)a.o + prow * D;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d0 = d * 32 + 8 * rq + 4 * g;  // this lane's 4 consecutive elements
          st16(op + d0, __builtin_bit_cast(u32x4, f32x4{oacc[d][4 * rq] * inv, oacc[d][4 * rq + 1] * inv,
                                                         oacc[d][4 * rq + 2] * inv, oacc[d][4 * rq + 3] * inv}));
        }
      }
      if (g == 0) st8(a.ml + prow * 2, __builtin_bit_cast(u32x2, f32x2{m_run, l_tot}));
    }
#pragma unroll
    for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
    m_run = NEG_INF;
    l_run = 0.f;
  };

  // The K and V tiles the compute below reads (set per tile; constant after unrolling).
  const uint8_t* Ks = lds_st0;
  const uint8_t* Vs = lds_st0 + TILE_BYTES;
  // MFMA A operands from LDS (FP8 widened to E on the way)
  auto k_operand = [&](int kb, int s) __attribute__((always_inline)) {
    if constexpr (IS_FP8) {
      const u32x2 raw = ld8(Ks + kb * 32 * D + koffs8[s]);
      const u32x2 lo = fp8x4_to_e<E>(raw[0]), hi = fp8x4_to_e<E>(raw[1]);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    } else {
      return ld16((const uint16_t*)Ks + kb * 32 * D + koffs[s]);
    }
  };
  auto v_operand = [&](int kb, int h, int d) __attribute__((always_inline)) {
    if constexpr (IS_FP8) {
      const u32x2 raw = lds_read_tr8(Vs + (kb * 32 + 16 * h) * D + voffs8[d]);
      const u32x2 lo = fp8x4_to_e<E>(raw[0]), hi = fp8x4_to_e<E>(raw[1]);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    } else {
      const uint16_t* vp = (const uint16_t*)Vs + (kb * 32 + 16 * h) * D;
      const u32x2 lo = lds_read_tr16(vp + voffs[d][0]);
      const u32x2 hi = lds_read_tr16(vp + voffs[d][1]);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };

  // S^T = K Q^T of one tile.
  auto tile_qk = [&](f32x16(&sacc)[KB]) __attribute__((always_inline)) {
    // The KB accumulation chains are independent; stepping them together keeps the MFMA
    // pipe fed while each chain's last result is in flight.
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) sacc[kb] = f32x16{};
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sacc[kb] = mfma32<E>(k_operand(kb, s), qf[s], sacc[kb]);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // Scale, mask, online softmax and O += V P of the tile at n0.
  auto tile_softmax_pv = [&](f32x16(&sacc)[KB], int n0) __attribute__((always_inline)) {
    // per-block score scale (FP8: times the block's k_scale, fp8.py:104)
    float sc[KB], vs[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if constexpr (KV::bytes == 1) {
        float ks, vsv;
        if constexpr (PAGED) {
          // the 64-key block of key n0 + 32 kb inside its page; keys at or past khi are
          // masked and pages outside the pool hold zero keys: scale 0 for both
          const int nk = n0 + kb * 32;
          const int page = nk < khi ? page_of(nk) : -1;
          const bool ok = (uint32_t)page < (uint32_t)a.num_pages;
          const int64_t at = ok ? (int64_t)page * a.ssb + (nk - slot_of(nk) * a.page_size) / 64 : 0;
          ks = ok ? ksc[at] : 0.f;
          vsv = ok ? vsc[at] : 0.f;
        } else {
          const int blk = (n0 + kb * 32) >> 6;  // 64-key FP8 scale block
          ks = ksc[blk];
          vsv = vsc[blk];
        }
        sc[kb] = fmaxf(c_abs * ks, kMinScale);
        vs[kb] = vsv;
      } else {
        sc[kb] = c_abs;
        vs[kb] = 1.f;
      }
    }
    // FP8: the factor folded into P.  Tiles start at multiples of 64 keys and hold at most 64,
    // so vs[0] is the tile's one V block scale (0 for keys outside the pool, which are zero
    // keys: then nothing is folded in and nothing rescaled).
    float vfold = 1.f;
    if constexpr (IS_FP8) {
      static_assert(BN <= 64, "one FP8 scale block per tile");
      const float vb = vs[0];
      if (vb > 0.f && !(vb <= 2.f * v_cur && v_cur <= 2.f * vb)) {
        // re-express O in this block's scale (O is 0 while v_cur is still 0)
        const float ratio = v_cur / vb;
#pragma unroll
        for (int d = 0; d < DB; ++d) oacc[d] *= ratio;
        v_cur = vb;
      }
      vfold = v_cur > 0.f ? vb / v_cur : 0.f;
    }

    // Masked tiles (the causal diagonal, the key tail) set excluded scores to -inf
    // in one uniform block; exp2 then gives 0 for them, so the softmax below is the
    // same straight-line code for every tile.
    if (n0 + BN > mask_from) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int n = n0 + kb * 32 + 16 * (r >> 3) + 8 * g + (r & 7);
          const bool ok = (n < khi) & ((a.causal == 0) | (n <= qlim));
          sacc[kb][r] = ok ? sacc[kb][r] : NEG_INF;
        }
      }
    }

    // tile max of the scaled scores (sc > 0: max of sc*s is sc*max(s))
    float mt = NEG_INF;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      float mx = sacc[kb][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = vmax(mx, sacc[kb][r]);
      mt = vmax(mt, mx * sc[kb]);
    }
    mt = max_xor32(mt);

    // Lazy rescale: keep the running max unless some row of the wave grew by
    // more than 2^8; p = 2^(c*s - m_run) then stays <= 256 (no overflow risk),
    // and O, l stay consistent because both use the same m_run.
    const float m_new = vmax(m_run, mt);
    if (__builtin_amdgcn_ballot_w64(m_new > m_run + kRescaleLog2) != 0) {
      const float m_safe_new = (m_new == NEG_INF) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_safe_new);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d) oacc[d] *= alpha;
      m_run = m_new;
    }
    const float m_safe = (m_run == NEG_INF) ? 0.f : m_run;

    // P = 2^(c*s - m) as 16-bit B operands of PV
    u32x4 pf[KB][2];
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fast_exp2(__builtin_fmaf(sacc[kb][r], sc[kb], -m_safe));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (KV::bytes == 1) {
          // v_scale / v_cur folded into P (v_cur is restored when the partial is emitted); the
          // row sum takes the unscaled fp32 P, as the reference's tl.sum(p, 1) (fp8.py:113)
          const float v = vfold;
#pragma unroll
          for (int e = 0; e < 8; ++e) rs += p[8 * h + e];
          pf[kb][h] = u32x4{pack2<E>(p[8 * h + 0] * v, p[8 * h + 1] * v), pack2<E>(p[8 * h + 2] * v, p[8 * h + 3] * v),
                            pack2<E>(p[8 * h + 4] * v, p[8 * h + 5] * v), pack2<E>(p[8 * h + 6] * v, p[8 * h + 7] * v)};
        } else {
          pf[kb][h] = u32x4{pack2<E>(p[8 * h + 0], p[8 * h + 1]), pack2<E>(p[8 * h + 2], p[8 * h + 3]),
                            pack2<E>(p[8 * h + 4], p[8 * h + 5]), pack2<E>(p[8 * h + 6], p[8 * h + 7])};
          // the row sum of the rounded P that the MFMA consumes (so O/l is a convex combination)
#pragma unroll
          for (int e = 0; e < 4; ++e) rs = sum2<E>(pf[kb][h][e], rs);
        }
      }
    }
    l_run += rs;

    // O^T += V^T P^T
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {  // DB independent chains per 16-key step
          oacc[d] = mfma32<E>(v_operand(kb, h, d), pf[kb][h], oacc[d]);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  if constexpr (STAGES == 2 && NW > 1) {
    // Multi-wave workgroups (speculative decode rows): two tiles in flight.  Tile t+2 is
    // issued into tile t's stage as soon as every wave has read it.  Every step issues its
    // refill, past the last tile with a zero-length descriptor (no memory access; the DMA
    // writes zeros into a stage nothing reads), so each wait is the same count: loads land
    // in issue order, and vmcnt <= 2*QPW after tile t+2's 2*QPW instructions means tile t+1
    // landed.  The barriers carry no memory fence (__syncthreads' fence would wait for
    // vmcnt(0)).  Measured on the 32k-key cache at n_q=16: +1.2% at 128-key partitions, +3.4%
    // at 4096; one-wave workgroups (n_q=1) lost 1.3% with it and keep one tile in flight.
    load_tile(klo, lds_st0);
    load_tile(klo + BN, lds_st1);
    vm_wait<2 * QPW>();
    wg_barrier<NW>();

    // One tile: S^T, softmax, O += P V on this stage, then refill it with tile t+2.  The
    // stage is a compile-time choice (the loop below is unrolled by 2).
    auto tile_step = [&](auto stage_tag, int t) __attribute__((always_inline)) {
      constexpr int ST = decltype(stage_tag)::value;
      uint8_t* cur = ST == 0 ? lds_st0 : lds_st1;
      const int n0 = klo + t * BN;
      if (wave_active && n0 < wave_khi) {
        Ks = cur;
        Vs = cur + TILE_BYTES;
        f32x16 sacc[KB];
        tile_qk(sacc);
        tile_softmax_pv(sacc, n0);
      }
      lgkm_wait0();  // this wave's reads of the stage have returned
      wg_barrier<NW>();
      load_tile(n0 + 2 * BN, cur);
      vm_wait<2 * QPW>();  // tile t+1 landed; tile t+2 stays in flight
      wg_barrier<NW>();
      // The last tile of a partition closes it.  Its stores are issued after this
      // tile's wait, so they complete under the next tile instead of stalling this one.
      if ((t + 1) % tiles_per_part == 0 || t + 1 == n_tiles) emit_partial(part0 + t / tiles_per_part);
    };
    for (int t = 0; t < n_tiles; t += 2) {
      tile_step(std::integral_constant<int, 0>{}, t);
      if (t + 1 < n_tiles) tile_step(std::integral_constant<int, 1>{}, t + 1);
    }
    lds_dma_wait();  // the zero-length refills past the end land before the workgroup ends
  } else if constexpr (STAGES == 2) {
    if (n_tiles > 0) load_tile(klo, lds_st0);
    lds_dma_wait();
    __syncthreads();

    // One tile: prefetch tile t+1 into the other stage, then S^T, softmax, O += P V on
    // this stage.  The stage is a compile-time choice (the loop below is unrolled by 2).
    auto tile_step = [&](auto stage_tag, int t) __attribute__((always_inline)) {
      constexpr int ST = decltype(stage_tag)::value;
      uint8_t* cur = ST == 0 ? lds_st0 : lds_st1;
      uint8_t* nxt = ST == 0 ? lds_st1 : lds_st0;
      const int n0 = klo + t * BN;
      if (t + 1 < n_tiles) load_tile(n0 + BN, nxt);  // released by the previous barrier
      if (wave_active && n0 < wave_khi) {
        Ks = cur;
        Vs = cur + TILE_BYTES;
        f32x16 sacc[KB];
        tile_qk(sacc);
        tile_softmax_pv(sacc, n0);
      }
      if (t + 1 < n_tiles) lds_dma_wait();
      __syncthreads();
      // The last tile of a partition closes it.  Its stores are issued after this
      // tile's wait: vmcnt counts stores too, so they complete under the next tile
      // instead of stalling this one.
      if ((t + 1) % tiles_per_part == 0 || t + 1 == n_tiles) emit_partial(part0 + t / tiles_per_part, cur);
    };
    for (int t = 0; t < n_tiles; t += 2) {
      tile_step(std::integral_constant<int, 0>{}, t);
      if (t + 1 < n_tiles) tile_step(std::integral_constant<int, 1>{}, t + 1);
    }
  } else {
    // Single stage: K_{t+1} is fetched as soon as S_t has been computed, V_{t+1} as soon
    // as O has taken V_t, so about one tile is in flight while the other half is read.
    // vmcnt counts this wave's loads and stores in issue order: waiting for it to drop
    // to QPW leaves only the QPW DMA instructions issued last in flight.
    Ks = lds_k1;
    Vs = lds_v1;
    if (n_tiles > 0) load_parts(klo, lds_k1, lds_v1, true, true);
    lds_dma_wait();
    __syncthreads();
    for (int t = 0; t < n_tiles; ++t) {
      const int n0 = klo + t * BN;
      const bool act = wave_active && n0 < wave_khi;
      vm_wait<QPW>();  // K_t landed (issued before V_t's QPW instructions)
      __syncthreads();
      f32x16 sacc[KB];
      if (act) tile_qk(sacc);
      if (t + 1 < n_tiles) {
        lgkm_wait0();  // this wave's K reads have returned
        __syncthreads();
        load_parts(n0 + BN, lds_k1, lds_v1, true, false);
        vm_wait<QPW>();  // V_t landed (issued before K_{t+1}'s QPW instructions)
      } else {
        lds_dma_wait();
      }
      __syncthreads();
      if (act) tile_softmax_pv(sacc, n0);
      if ((t + 1) % tiles_per_part == 0 || t + 1 == n_tiles) emit_partial(part0 + t / tiles_per_part);
      if (t + 1 < n_tiles) {
        lgkm_wait0();  // this wave's V reads have returned
        __syncthreads();
        load_parts(n0 + BN, lds_k1, lds_v1, false, true);
      }
    }
  }

  // partitions past the visible keys (causal, or past the sequence end): empty
  // partials, m = -inf and l = 0, which the combine weighs by zero
  for (int part = part0 + (n_tiles + tiles_per_part - 1) / tiles_per_part; part < part_end; ++part) emit_partial(part);
}

// Log-sum-exp merge of split-K partials (triton_splitk.py:99-127), with each fp32 partial
// O_s stored normalised (O_s = un-normalised partial / l_s):
//   m = max_s m_s;  w_s = 2^(m_s - m) l_s;  O = sum_s w_s O_s / sum_s w_s   (0 when the sum is 0)
// One 256-thread workgroup per output row; D/8 threads cover a partial row with two 16-byte
// loads each (8 elements), so 256/(D/8) partials are read concurrently.  Each thread merges
// its partials online (running max, rescaled sums), and the threads' (m, l, acc) triples
// are merged through LDS at the end: one pass over the partials, no separate max pass.
template <int D, class E, bool PART_MAJOR>
__global__ void __launch_bounds__(256) splitk_combine_kernel(const CombineArgs c) {
  constexpr int TPS = D / 8;
  constexpr int SPB = 256 / TPS;
  constexpr float NEG_INF = -__builtin_inff();
  __shared__ f32x4 part[SPB][TPS][2];
  __shared__ f32x2 mlpart[SPB];

  const int64_t row = blockIdx.x;  // (b, hq, qi) flattened
  const int S = c.n_split;
  // row-major partials: S consecutive rows; partition-major: one row of each of S blocks of
  // R = G * Nq rows (the grid has fewer than 2^31 rows: 32-bit index arithmetic)
  int64_t base = row * S, pstride = 1;
  if constexpr (PART_MAJOR) {
    const uint32_t r32 = (uint32_t)row, nq = (uint32_t)c.nq, grp = (uint32_t)c.group;
    const uint32_t bh = r32 / nq, qrow = r32 - bh * nq;  // (b * Hq + hq), qi
    const uint32_t bkv = bh / grp, gi = bh - bkv * grp;  // (b * Hkv + kvh), q-head in group
    pstride = (int64_t)grp * nq;
    base = (int64_t)bkv * S * pstride + (int64_t)gi * nq + qrow;
  }
  const float* ml = c.ml + base * 2;
  const float* op = c.opart + base * D;
  const int tid = (int)threadIdx.x;
  const int sg = tid / TPS, dq = tid % TPS;

  // Online merge of partials sg, sg + SPB, ...: (m, l, acc) with acc and l relative to 2^m.
  // An empty partial (m_s = -inf, l_s = 0) gets weight 0; m stays -inf until a partial
  // with keys arrives, and the -inf guards keep 2^(-inf - -inf) out of the sums.
  // Partials are loaded CH at a time before any is merged, so that CH loads per thread are in
  // flight at once (the compiler kept a load-then-merge loop at one load in flight; measured:
  // the D=256 decode merge over 256 partitions went from 13.0 to 8.9 us, the D=128 merges
  // did not change).  Slots past the last partial take the empty partial (m = -inf, l = 0),
  // which merges as a no-op.
  constexpr int CH = 8;
  float m = NEG_INF, l = 0.f;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = sg; s0 < S; s0 += CH * SPB) {
    f32x2 st[CH];
    f32x4 pv0[CH], pv1[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int s = s0 + u * SPB;
      if (s < S) {
        st[u] = __builtin_bit_cast(f32x2, ld8(ml + 2 * s * pstride));
        pv0[u] = __builtin_bit_cast(f32x4, ld16(op + s * pstride * D + 8 * dq));
        pv1[u] = __builtin_bit_cast(f32x4, ld16(op + s * pstride * D + 8 * dq + 4));
      } else {
        st[u] = f32x2{NEG_INF, 0.f};
        pv0[u] = pv1[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const float m_new = fmaxf(m, st[u][0]);
      const float m_ref = (m_new == NEG_INF) ? 0.f : m_new;
      const float alpha = fast_exp2(m - m_ref);  // 0 while m = -inf
      const float w = fast_exp2(st[u][0] - m_ref) * st[u][1];
      l = l * alpha + w;
      acc0 = acc0 * alpha + w * pv0[u];
      acc1 = acc1 * alpha + w * pv1[u];
      m = m_new;
    }
  }
  part[sg][dq][0] = acc0;
  part[sg][dq][1] = acc1;
  if (dq == 0) mlpart[sg] = f32x2{m, l};
  __syncthreads();
  if (tid < TPS) {
    float mx = NEG_INF;
#pragma unroll
    for (int k = 0; k < SPB; ++k) mx = fmaxf(mx, mlpart[k][0]);
    const float m_ref = (mx == NEG_INF) ? 0.f : mx;
    f32x4 t0 = {0.f, 0.f, 0.f, 0.f}, t1 = {0.f, 0.f, 0.f, 0.f};
    float lt = 0.f;
#pragma unroll 4
    for (int k = 0; k < SPB; ++k) {
      const float a = fast_exp2(mlpart[k][0] - m_ref);
      lt += a * mlpart[k][1];
      t0 += a * part[k][tid][0];
      t1 += a * part[k][tid][1];
    }
    const float l_safe = (lt == 0.f) ? 1.f : lt;
    const float inv = 1.f / l_safe;
    const int qi = (int)(row % c.nq);
    const int64_t bh = row / c.nq;
    const int hq = (int)(bh % c.hq);
    const int64_t b = bh / c.hq;
    // natural-log LSE of the row (triton_fwd.py:169-172): m and the weights are relative to 2^m_ref
    if (c.lse != nullptr && tid == 0) c.lse[b * c.slb + (int64_t)hq * c.slh + qi] = (mx + __log2f(l_safe)) * kLn2;  // -inf for a row without keys, as the prefill kernel
    uint16_t* o = (uint16_t*)c.o + b * c.sob + (int64_t)hq * c.soh + (int64_t)qi * c.son + 8 * tid;
    st8(o, u32x2{pack2<E>(t0[0] * inv, t0[1] * inv), pack2<E>(t0[2] * inv, t0[3] * inv)});
    st8(o + 4, u32x2{pack2<E>(t1[0] * inv, t1[1] * inv), pack2<E>(t1[2] * inv, t1[3] * inv)});
  }
}

// ------------------------------------------------------------------------------------
// Host-side launchers
// ------------------------------------------------------------------------------------

template <int D, class E, class KV, int NW, int BN, bool PAGED, bool ONE_STAGE = false>
static hipError_t launch_splitk(const TileArgs& a, hipStream_t stream) {
  // paged pools of 16 + 32k keys per page take 16-key page groups (twice the descriptors)
  if constexpr (PAGED && KV::bytes == 2) {
    if (a.page_size % 32 != 0) {
      hipLaunchKernelGGL((attn_splitk_kernel<D, E, KV, NW, BN, PAGED, ONE_STAGE, 16>), dim3((unsigned)a.total),
                         dim3(NW * 64), 0, stream, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((attn_splitk_kernel<D, E, KV, NW, BN, PAGED, ONE_STAGE, 32>), dim3((unsigned)a.total),
                     dim3(NW * 64), 0, stream, a);
  return hipGetLastError();
}

template <int D, class E>
static hipError_t launch_combine(const CombineArgs& c, int64_t rows, hipStream_t stream) {
  // the layout is a template argument: with a runtime stride the row-major merge ran 30-45% slower
  if (c.part_major) {
    hipLaunchKernelGGL((splitk_combine_kernel<D, E, true>), dim3((unsigned)rows), dim3(256), 0, stream, c);
  } else {
    hipLaunchKernelGGL((splitk_combine_kernel<D, E, false>), dim3((unsigned)rows), dim3(256), 0, stream, c);
  }
  return hipGetLastError();
}

TileArgs common_args(const fa_fwd_params& p) {
  TileArgs a{};
  a.q = p.q;
  a.k = p.k;
  a.v = p.v;
  a.sqb = p.q_stride_b;
  a.sqh = p.q_stride_h;
  a.sqn = p.q_stride_n;
  a.skb = p.k_stride_b;
  a.skh = p.k_stride_h;
  a.skn = p.k_stride_n;
  a.svb = p.v_stride_b;
  a.svh = p.v_stride_h;
  a.svn = p.v_stride_n;
  a.hq = p.heads_q;
  a.hkv = p.heads_kv;
  a.group = p.heads_q / p.heads_kv;
  a.nq = p.seqlen_q;
  a.nk = p.seqlen_k;
  a.qk_scale = p.scale * kLog2e;  // same fp32 product as triton_fwd.py:143
  a.causal = p.causal ? 1 : 0;
  a.k_scale = p.k_scale;
  a.v_scale = p.v_scale;
  a.ssb = p.scale_stride_b;
  a.ssh = p.scale_stride_h;
  return a;
}

int splitk_waves_for_rows(int rows) { return rows <= 32 ? 1 : (rows <= 64 ? 2 : 4); }

// Partitions per workgroup.  One partition per workgroup measured fastest on MI355X for
// one-wave 16-bit decode (fine-grained workgroups keep every CU's memory pipeline full to
// the end of the grid; two per workgroup: -3% at 128-key partitions).  Workgroups with
// less memory work per instruction stream (FP8 tiles, or row blocks of 2-4 waves) gain
// 2-2.4% from two partitions when the grid is fine (at least 16384 workgroups, 64 per CU);
// coarser grids keep one so that every CU stays busy.  Beyond that, several partitions per
// workgroup only cap the grid at kMaxWgs.  16-bit paged decode keeps one; FP8 pools follow the
// dense FP8 rule (run_splitk lowers it again if a workgroup's pages would not fit the
// block-table entries it holds), so a paged FP8 call decomposes as the dense one does.
int splitk_parts_per_wg(int64_t items, int n_split, bool fp8, int nw, bool paged) {
  constexpr int64_t kMaxWgs = int64_t{1} << 20, kFineGrid = int64_t{1} << 14;
  int64_t want = (items * n_split + kMaxWgs - 1) / kMaxWgs;
  if (!paged && (fp8 || nw > 1) && items * n_split >= kFineGrid) want = std::max<int64_t>(want, 2);
  return (int)std::max<int64_t>(1, std::min<int64_t>(want, n_split));
}

template <int D, class E, class KV, bool PAGED>
static hipError_t launch_split_nw(const TileArgs& a, int nw, hipStream_t stream) {
  switch (nw) {
    case 1:
      // Single LDS stage for 16-bit K/V where two stages cap the workgroups per CU by LDS
      // (measured on the 32k-key decode cache): D=64 (10 -> 16 per CU; +4.6% at 128-key
      // partitions, +1.4% at 4096), D=256 (2 -> 4; +15% at 128-key partitions) and D=128
      // with partitions of 512 keys or more (5 -> 8; +1.3-2.7%; at 128 keys the longer
      // per-tile wait costs 1.2% instead).  FP8 tiles are small enough already.
      if constexpr (KV::bytes == 2) {
        if (D != 128 || a.split_len >= 512) return launch_splitk<D, E, KV, 1, 32, PAGED, true>(a, stream);
      }
      return launch_splitk<D, E, KV, 1, 32, PAGED>(a, stream);
    case 2:
      return launch_splitk<D, E, KV, 2, 32, PAGED>(a, stream);
    default:  // 64-key tiles, but 32 at D=256 (a 16-bit K or V tile stays 16 KiB)
      return launch_splitk<D, E, KV, 4, (D == 256 ? 32 : 64), PAGED>(a, stream);
  }
}

template <int D, class E>
static hipError_t launch_split(const TileArgs& a, bool fp8, bool paged, int nw, hipStream_t stream) {
  if (paged) return fp8 ? launch_split_nw<D, E, FP8, true>(a, nw, stream) : launch_split_nw<D, E, E, true>(a, nw, stream);
  return fp8 ? launch_split_nw<D, E, FP8, false>(a, nw, stream) : launch_split_nw<D, E, E, false>(a, nw, stream);
}

// ------------------------------------------------------------------------------------
// Scratch for the entry point that allocates nothing (fa_attention_splitk_noalloc): the
// split-K workspace lives in a file-scope device array, one copy per GPU for the life of the
// process.  Host code may not use the array's name as a device address: each device's
// address comes from hipGetSymbolAddress, called once per device with that device current.
// ------------------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[kSplitkScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

fa_status splitk_scratch(void** ptr, const char** err) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, err);
  if (dev < 0 || dev >= kMaxDevices) {
    *err = "device index beyond the scratch table";
    return FA_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, err);
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return FA_OK;
}

fa_status run_splitk(const fa_fwd_params& p, int32_t split_len, void* workspace, hipStream_t stream,
                     const char** err, const fa_paged_kv* kv) {
  TileArgs a = common_args(p);
  if (kv != nullptr) {
    a.skb = a.svb = 0;
    a.block_table = kv->block_table;
    a.seqlens_k = kv->seqlens_k;
    a.sbt = kv->block_table_stride;
    a.spk = kv->k_page_stride;
    a.spv = kv->v_page_stride;
    a.page_size = kv->page_size;
    a.num_pages = kv->num_pages;
    int lg = 0;  // ceil(log2(page_size)); page_size <= 2^24 (C ABI)
    while ((int64_t{1} << lg) < (int64_t)kv->page_size) ++lg;
    a.page_magic_shift = 31 + lg;
    a.page_magic = (uint32_t)(((uint64_t{1} << a.page_magic_shift) + (uint64_t)kv->page_size - 1) / (uint64_t)kv->page_size);
  }
  if (p.batch <= 0 || p.seqlen_q <= 0) return FA_OK;
  const int S = p.seqlen_k > 0 ? (p.seqlen_k + split_len - 1) / split_len : 1;
  const int rows = a.group * p.seqlen_q;
  const int nw = splitk_waves_for_rows(rows);
  a.n_rowblk = (rows + nw * 32 - 1) / (nw * 32);
  a.n_split = S;
  a.split_len = split_len;
  const int64_t items = (int64_t)p.batch * p.heads_kv * a.n_rowblk;
  const bool fp8_kv = p.kv_dtype == FA_DTYPE_FP8_E4M3;
  a.ppw = splitk_parts_per_wg(items, S, fp8_kv, nw, kv != nullptr && !fp8_kv);
  if (kv != nullptr) {
    // a workgroup's keys span at most (ppw * split_len - 1) / page_size + 2 pages, and it
    // holds 256 block-table entries
    auto slots_for = [&](int ppw) { return ((int64_t)ppw * split_len - 1) / kv->page_size + 2; };
    while (a.ppw > 1 && slots_for(a.ppw) > 256) --a.ppw;
    const int64_t slots = slots_for(a.ppw);
    if (slots > 256) {
      *err = "split_len too long for the page size: a partition may span at most 256 pages";
      return FA_ERR_UNSUPPORTED;
    }
  }
  a.n_chunk = (S + a.ppw - 1) / a.ppw;
  const int64_t total = items * a.n_chunk;
  const int64_t out_rows = (int64_t)p.batch * p.heads_q * p.seqlen_q;
  if (total > INT32_MAX || out_rows > INT32_MAX) {
    *err = "grid too large";
    return FA_ERR_UNSUPPORTED;
  }
  a.total = (int32_t)total;
  a.o = workspace;  // fp32 partials (rows x S x D floats), then the (m, l) pairs (rows x S x 2)
  a.ml = (float*)((uint8_t*)workspace + out_rows * S * p.head_dim * 4);
  // With many partitions the partial writes are a real share of the traffic; partition-major
  // blocks then make each workgroup's writes contiguous (measured at 128-key partitions, end to
  // end: n_q=16 +3.0%, paged +1.8%, FP8 +3.1%, paged FP8 +14%, n_q=1 +0.2%).  With few, the
  // combine's reads of one row's partials stay contiguous in the row-major layout, and at D=256
  // partition-major measured 0.7% slower.
  a.part_major = (S >= 32 && p.head_dim <= 128) ? 1 : 0;
  const bool fp8 = p.kv_dtype == FA_DTYPE_FP8_E4M3;
  const bool bf = p.dtype == FA_DTYPE_BF16;
  hipError_t e = hipErrorInvalidValue;
  const bool paged = kv != nullptr;
  if (p.head_dim == 128) {
    e = bf ? launch_split<128, BF16>(a, fp8, paged, nw, stream) : launch_split<128, F16>(a, fp8, paged, nw, stream);
  } else if (p.head_dim == 64) {
    e = bf ? launch_split<64, BF16>(a, fp8, paged, nw, stream) : launch_split<64, F16>(a, fp8, paged, nw, stream);
  } else if (p.head_dim == 256) {
    e = bf ? launch_split<256, BF16>(a, fp8, paged, nw, stream) : launch_split<256, F16>(a, fp8, paged, nw, stream);
  }
  if (e != hipSuccess) return hip_status(e, err);

  CombineArgs c{};
  c.opart = (const float*)a.o;
  c.ml = a.ml;
  c.o = p.o;
  c.sob = p.o_stride_b;
  c.soh = p.o_stride_h;
  c.son = p.o_stride_n;
  c.hq = p.heads_q;
  c.group = p.heads_q / p.heads_kv;
  c.part_major = a.part_major;
  c.nq = p.seqlen_q;
  c.n_split = S;
  c.lse = p.lse;
  c.slb = p.lse_stride_b;
  c.slh = p.lse_stride_h;
  if (p.head_dim == 128) {
    e = bf ? launch_combine<128, BF16>(c, out_rows, stream) : launch_combine<128, F16>(c, out_rows, stream);
  } else if (p.head_dim == 256) {
    e = bf ? launch_combine<256, BF16>(c, out_rows, stream) : launch_combine<256, F16>(c, out_rows, stream);
  } else {
    e = bf ? launch_combine<64, BF16>(c, out_rows, stream) : launch_combine<64, F16>(c, out_rows, stream);
  }
  return hip_status(e, err);
}

}  // namespace fa
