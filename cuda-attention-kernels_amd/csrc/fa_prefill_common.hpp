// The workgroup -> (batch, q-head, row block) schedule of the 16-bit prefill kernel
// (fa_prefill.hip), kept apart from the kernel body.
#pragma once

#include "fa_device.hpp"
#include "fa_internal.hpp"

namespace fa {

struct PrefillItem {
  int b;    // batch (varlen: sequence)
  int hq;   // q-head
  int kvh;  // kv-head
  int rb;   // row block (NW * rows-per-wave queries)
};

// Workgroup blockIdx.x -> work item; false for grid padding (varlen), uniform over the workgroup.
//
// Dense: scheduling units are the q-heads of as many kv-heads as keep about unit_bytes of
// K/V (prefill_unit_bytes; one XCD's L2 is 4 MB).  Units follow each other in logical order, and
// xcd_remap hands each XCD a contiguous range of logical indices, so an XCD works through one
// or two units at a time and re-reads K/V from its L2.  Inside a unit the query blocks go by
// rank, heaviest causal blocks first, all heads of the unit at each rank, which keeps the
// XCD's CUs evenly loaded to the end.
//
// Varlen: sequences differ in length, and ranges of whole sequences per XCD load the XCDs
// unevenly (measured: a 16-sequence batch ran at 0.18 of peak).  There the order is
// rank-major per XCD: the dispatcher deals workgroups to the XCDs round-robin (blockIdx % 8),
// XCD x takes the (sequence, kv-head) groups g = x (mod 8) and walks them rank by rank,
// heaviest causal ranks first, with the q-heads of one kv-head side by side, so they run
// together and read its K/V through one L2 (measured: +8-10% over rank-major across all
// XCDs, which fetched each K/V tile into up to four L2s).  The host pads the grid to a
// multiple of 8 groups; padding returns false.

// K/V bytes of the q-heads one dense scheduling unit holds.  At D=128 half an XCD's L2: the
// Q and O streams (64 KiB each per 256-row workgroup) pass through the same L2, and a unit
// whose K/V filled all 4 MB had them evicted and re-fetched (causal GQA B=4 Hq=32 Hkv=8 N=4096:
// 296 MB read for 201 MB of Q, K and V with 4 MB units, 216 MB with 2 MB units, at the same
// speed).  At D <= 64 a workgroup's Q and O are half as large or less, and halving the unit
// cost 2-8% (MHA D=64 N=4096: fewer heads to spread over the XCD's CUs), so those keep 4 MB.
inline int64_t prefill_unit_bytes(int head_dim) { return int64_t{head_dim == 128 ? 2 : 4} << 20; }

// q-heads per dense scheduling unit: the q-heads of as many whole kv-heads as fit
// prefill_unit_bytes.  The host computes it once per launch (TileArgs::u_heads).
inline int prefill_unit_heads(int nk, int head_dim, int group) {
  const int64_t kv_head_bytes = (int64_t)(nk > 1 ? nk : 1) * head_dim * 2 * 2;
  const int64_t kv_heads = prefill_unit_bytes(head_dim) / kv_head_bytes;
  return (int)(kv_heads > 1 ? kv_heads : 1) * group;
}

template <int D>
__device__ __forceinline__ bool prefill_item(const TileArgs& a, PrefillItem& it) {
  // Every quantity here is non-negative: unsigned division needs no sign fix-ups, and all
  // waves of the workgroup run this scalar code before their first DMA.
  constexpr uint32_t kXcds = 8;
  const uint32_t group = (uint32_t)a.group, bid = blockIdx.x;
  uint32_t mrev, item;
  if (a.varlen) {
    const uint32_t xcd = bid % kXcds, local = bid / kXcds;
    const uint32_t per_rank = (uint32_t)a.total / ((uint32_t)a.n_rowblk * kXcds);  // this XCD's items per rank
    mrev = local / per_rank;
    const uint32_t j = local - mrev * per_rank;
    const uint32_t jg = j / group;
    const uint32_t kvg = jg * kXcds + xcd;
    if (kvg >= (uint32_t)a.kv_groups) return false;
    item = kvg * group + (j - jg * group);
  } else {
    const uint32_t nbh = (uint32_t)a.kv_groups * group;  // (batch, q-head) pairs
    const uint32_t logical = (uint32_t)xcd_remap((int)bid, a.total);
    const uint32_t unit_heads = (uint32_t)a.u_heads;  // prefill_unit_heads(nk, D, group)
    const uint32_t unit = logical / (uint32_t)a.u_items;
    const uint32_t within = logical - unit * (uint32_t)a.u_items;
    const uint32_t unit_size = min(unit_heads, nbh - unit * unit_heads);
    mrev = within / unit_size;
    item = unit * unit_heads + (within - mrev * unit_size);
  }
  const uint32_t kvi = item / group;
  const uint32_t gi = item - kvi * group;
  const uint32_t bb = kvi / (uint32_t)a.hkv;
  it.kvh = (int)(kvi - bb * (uint32_t)a.hkv);
  it.b = (int)bb;
  it.hq = it.kvh * a.group + (int)gi;
  it.rb = a.causal ? (a.n_rowblk - 1 - (int)mrev) : (int)mrev;  // heaviest causal blocks first
  return true;
}

}  // namespace fa
