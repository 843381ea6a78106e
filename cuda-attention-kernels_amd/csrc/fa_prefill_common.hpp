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
// Dense: scheduling units are the q-heads of as many kv-heads as keep about kL2UnitBytes of
// K/V (one XCD's L2 is 4 MB).  Units follow each other in logical order, and xcd_remap hands
// each XCD a contiguous range of logical indices, so an XCD works through one or two units at
// a time and re-reads K/V from its L2.  Inside a unit the query blocks go by rank, heaviest
// causal blocks first, all heads of the unit at each rank, which keeps the XCD's CUs evenly
// loaded to the end.
//
// Varlen: sequences differ in length, and ranges of whole sequences per XCD load the XCDs
// unevenly (measured: a 16-sequence batch ran at 0.18 of peak).  There the order is
// rank-major per XCD: the dispatcher deals workgroups to the XCDs round-robin (blockIdx % 8),
// XCD x takes the (sequence, kv-head) groups g = x (mod 8) and walks them rank by rank,
// heaviest causal ranks first, with the q-heads of one kv-head side by side, so they run
// together and read its K/V through one L2 (measured: +8-10% over rank-major across all
// XCDs, which fetched each K/V tile into up to four L2s).  The host pads the grid to a
// multiple of 8 groups; padding returns false.
template <int D>
__device__ __forceinline__ bool prefill_item(const TileArgs& a, PrefillItem& it) {
  constexpr int64_t kL2UnitBytes = int64_t{4} << 20;
  constexpr int kXcds = 8;
  int mrev, item;
  if (a.varlen) {
    const int xcd = (int)blockIdx.x % kXcds, local = (int)blockIdx.x / kXcds;
    const int per_rank = a.total / (a.n_rowblk * kXcds);  // this XCD's (group, q-head) items per rank
    mrev = local / per_rank;
    const int j = local % per_rank;
    const int kvg = (j / a.group) * kXcds + xcd;
    if (kvg >= a.kv_groups) return false;
    item = kvg * a.group + j % a.group;
  } else {
    const int nbh = a.total / a.n_rowblk;  // (batch, q-head) pairs
    const int logical = xcd_remap((int)blockIdx.x, a.total);
    const int64_t kv_head_bytes = (int64_t)max(a.nk, 1) * D * 2 * 2;
    const int unit_heads = max(1, (int)(kL2UnitBytes / kv_head_bytes)) * a.group;
    const int unit = logical / (unit_heads * a.n_rowblk);
    const int within = logical % (unit_heads * a.n_rowblk);
    const int unit_size = min(unit_heads, nbh - unit * unit_heads);
    mrev = within / unit_size;
    item = unit * unit_heads + within % unit_size;
  }
  const int gi = item % a.group;
  item /= a.group;
  it.kvh = item % a.hkv;
  it.b = item / a.hkv;
  it.hq = it.kvh * a.group + gi;
  it.rb = a.causal ? (a.n_rowblk - 1 - mrev) : mrev;  // heaviest causal blocks first
  return true;
}

}  // namespace fa
