// Software-pipelined FlashAttention-2 prefill kernel for MI355X (gfx950).
//
// Serves the reference's dense and varlen prefill, attn_fwd_mma_kernel
// (csrc/flash_attn_mma.cu:63-242) and _attn_fwd_kernel
// (fused_attn/triton_fwd.py:85-172), for 16-bit Q/K/V with D in {16, 32, 64, 128, 256}.
//
// A workgroup of NW waves (8 for D=128 from 4096 queries, 2048 without the causal mask,
// otherwise 4) covers NW*32 queries of one
// q-head; wave w owns 32 of them.  K and V stream through LDS in 64-key tiles (128 at D <= 64,
// 32 at D=256), each in two buffers filled
// straight from memory (buffer_load ... lds).  The product order per wave is the
// same as in the split-K kernel (S^T = K Q^T with the softmax lane-local,
// P^T kept in VGPRs as the B operand of O^T += V^T P^T), but the loop is
// software-pipelined so that one wave always has matrix work and vector work
// that do not depend on each other:
//
//   iteration t:  S_{t+1} = K_{t+1} Q^T            (MFMA)
//                 P_t = 2^(c S_t - m), row sums    (VALU, exp)
//                 O^T += V_t^T P_t^T               (MFMA)
//                 max of S_{t+1}                   (VALU)
//
// MFMA and VALU instructions of one wave overlap when they are interleaved in
// its own instruction stream; a wave that only issues MFMAs while another wave
// of the SIMD only issues VALU work overlaps much less.  K therefore runs one
// tile ahead of V: during iteration t the buffers hold K_{t+1} and V_t while
// K_{t+2} and V_{t+1} are in flight into the other buffers.
//
// Element-wise masking is needed only on the causal diagonal and the key tail; it
// sits behind a uniform branch after the main block, so an iteration is one basic
// block apart from that and the rare online-softmax rescale.
//
// A workgroup's start and end are kept short: the first tiles' DMA goes out before Q
// and before the rest of the set-up, and the output is written through LDS in whole rows.
#include <float.h>

#include <algorithm>

#include <type_traits>

#include "fa_device.hpp"
#include "fa_internal.hpp"
#include "fa_prefill_common.hpp"
#include "fa_tile.hpp"

namespace fa {

// Compile-time loop: f(integral_constant<int, I>) for I in [I0, N), always fully unrolled.
template <int I0, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I0 < N) {
    f(std::integral_constant<int, I0>{});
    static_for<I0 + 1, N>(f);
  }
}

template <int D, class E, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2)))
attn_fwd_kernel(const TileArgs a) {
  // 64-key tiles at D=128, 128-key tiles at D=64, 32-key tiles at D=256: 16 KiB per K (or V)
  // tile and 32 MFMAs per iteration (measured: D=64 prefill 3% faster than with 64-key
  // tiles).  D=32 and D=16 keep 128-key tiles: the scores of a tile already take 64 registers
  // per lane.  At D=256 the fp32 output accumulator alone takes 128 registers per lane, so the
  // kernel runs one wave per SIMD there.
  constexpr int BN = D <= 64 ? 128 : (D == 256 ? 32 : 64);
  static_assert(NW == 4 || (NW == 8 && D != 256), "4 or 8 waves (two per SIMD) per workgroup");
  // V tiles are at least 32 columns wide, since O^T += V^T P^T works in 32-wide d blocks.  At
  // D=16 the upper 16 columns of a V row in LDS repeat the lower ones (the DMA reads each source
  // chunk twice); they feed only O^T rows 16..31, which are never stored.
  constexpr int DV = D < 32 ? 32 : D;
  using Shape = TileShape<D, BN>;    // K tiles
  using VShape = TileShape<DV, BN>;  // V tiles
  constexpr int TILE = Shape::TILE, VTILE = VShape::TILE;
  constexpr int KB = BN / 32;  // 32-key MFMA blocks per tile
  constexpr int KS = D / 16;   // k-steps of S^T = K Q^T
  constexpr int DB = DV / 32;  // 32-wide d blocks of O^T
  constexpr int QPW = (TILE * 2 / 1024) / NW;    // 1-KiB DMA blocks per wave per K tile
  constexpr int VQPW = (VTILE * 2 / 1024) / NW;  // and per V tile
  static_assert(D == 16 || D == 32 || D == 64 || D == 128 || D == 256, "head dim");
  static_assert((TILE * 2) % (1024 * NW) == 0 && (VTILE * 2) % (1024 * NW) == 0,
                "direct loads must split evenly over the waves");
  constexpr float NEG_INF = -__builtin_inff();
  // At D=16 the loop is bound by its vector work (the two products cost 12 MFMAs per 128-key
  // tile against about 200 VALU instructions), so the row sums of P move to the matrix core: one
  // 16x16x32 MFMA per 16-key half-block against a 0/1 operand (rowsum_ones) replaces eight
  // v_dot2 per tile and wave (measured +5.6% at B=4 H=16 N=4096 causal; no gain at D >= 32,
  // and at D=64 the extra registers spill).
  constexpr bool MFMA_ROWSUM = D == 16;

  // Four separate arrays: every access names its buffer at compile time, so the
  // compiler can tell that a DMA into one buffer never aliases reads of another.
  __shared__ __align__(16) uint16_t k_buf0[TILE];
  __shared__ __align__(16) uint16_t k_buf1[TILE];
  __shared__ __align__(16) uint16_t v_buf0[VTILE];
  __shared__ __align__(16) uint16_t v_buf1[VTILE];

  // ---- work item: (batch, q-head, NW*32-query block) ----------------------------------
  // One scalar load per 64-byte line of the argument block, all issued at entry: left to the
  // compiler, the fields are loaded where they are first used, in four dependent round trips
  // before the first DMA can go out.
  {
    const uint32_t* ap = reinterpret_cast<const uint32_t*>(&a);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(TileArgs) / 4); i += 16) {
      const uint32_t x = ap[i];
      __asm__ volatile("" ::"s"(x));
    }
  }
  PrefillItem it;
  if (!prefill_item<D>(a, it)) return;  // grid padding (uniform over the workgroup)
  const int b = it.b, hq = it.hq, kvh = it.kvh, rb = it.rb;

  int seq_q = a.nq, seq_k = a.nk;
  int64_t qtok0 = 0, ktok0 = 0;
  if (a.varlen) {
    // the offsets are the same for every lane: keep them (and all addresses derived
    // from them) in scalar registers
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
  if (a.causal) khi = min(khi, min(r0 + NW * 32, seq_q) - 1 + offset + 1);
  const int n_tiles = khi > 0 ? (khi + BN - 1) / BN : 0;
  // Tiles [0, n_fast) hold only keys that every query of the workgroup sees.
  const int wg_mask_from = a.causal ? min(khi, r0 + offset + 1) : khi;
  const int n_fast = wg_mask_from > 0 ? wg_mask_from / BN : 0;

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
  // Key tiles with a key visible to some row of this wave.  Causal: the wave's rows may end
  // before the workgroup's last row, and its later tiles hold only -inf scores (P = 0), so the
  // wave skips their compute and only issues its share of the DMA (with 8 waves up to 3 tiles).
  const int wave_khi = a.causal ? min(khi, min(wr0 + 32, seq_q) - 1 + offset + 1) : khi;
  const int wave_tiles = wave_khi > 0 ? (wave_khi + BN - 1) / BN : 0;
  const int qlim = qi + offset;  // last key this lane's row may see (causal)

  const uint8_t* kbase = (const uint8_t*)a.k + ((int64_t)b * a.skb + (int64_t)kvh * a.skh + ktok0 * a.skn) * 2;
  const uint8_t* vbase = (const uint8_t*)a.v + ((int64_t)b * a.svb + (int64_t)kvh * a.svh + ktok0 * a.svn) * 2;
  const int64_t krow_bytes = a.skn * 2, vrow_bytes = a.svn * 2;

  // A negative softmax scale is applied by negating Q (exact for 16-bit floats), so
  // the kernel works with c = |scale| * log2(e) > 0 and max(c*s) = c*max(s).  c is
  // kept away from 0 so that a masked score (-inf) times c stays -inf.
  const uint32_t qsign = a.qk_scale < 0.f ? 0x80008000u : 0u;
  const float c = fmaxf(fabsf(a.qk_scale), kMinScale);

  // ---- Q fragments (B operand of S^T), resident for the whole kernel ----------------
  // (rows past the end read row 0, which exists, and are zeroed).  They are loaded right
  // after the first K/V tiles' DMA is issued, so that both latencies overlap, and fixed up
  // (sign, rows past the end) only once the rest of the set-up is done.
  u32x4 qf[KS];
  auto load_q = [&]() __attribute__((always_inline)) {
    const int64_t qrow = qtok0 + (row_ok ? qi : 0);
    const uint16_t* qp = (const uint16_t*)a.q + (int64_t)b * a.sqb + (int64_t)hq * a.sqh + qrow * a.sqn + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = ld16(qp + 16 * s);
  };

  // ---- K/V tiles: global -> LDS --------------------------------------------------------
  // Buffer loads past the byte limit return zeros, which zero-fills the keys >= khi of
  // the last tile (masked keys must not carry NaN/Inf into P*V).  The limit fits 32 bits
  // (row stride checked at the C ABI) and is wave-uniform, so descriptors live in SGPRs.
  auto limit = [&](int n0, int64_t row_bytes) __attribute__((always_inline)) {
    const int valid = min(khi - n0, BN);
    return __builtin_amdgcn_readfirstlane(valid > 0 ? (uint32_t)(valid - 1) * (uint32_t)row_bytes + (uint32_t)(D * 2)
                                                    : 0u);
  };
  // Tile descriptors (a tile past khi gets a zero-length one: its DMA writes zeros) and
  // the wave's i-th 1-KiB DMA instruction of a K or V tile.
  auto k_rsrc = [&](int n0) __attribute__((always_inline)) { return make_rsrc(kbase + (int64_t)n0 * krow_bytes, limit(n0, krow_bytes)); };
  auto v_rsrc = [&](int n0) __attribute__((always_inline)) { return make_rsrc(vbase + (int64_t)n0 * vrow_bytes, limit(n0, vrow_bytes)); };
  auto dma_k = [&](const __amdgpu_buffer_rsrc_t& rk, uint16_t* dst, int i) __attribute__((always_inline)) {
    const int blk = wave * QPW + i;
    const int byte = blk * 1024 + lane * 16;
    const int r = byte / (D * 2), p = (byte % (D * 2)) / 16;
    lds_dma16<false>(rk, (uint8_t*)dst + blk * 1024, kperm(r) * (int)krow_bytes + ((p ^ Shape::swz_k(r)) * 16));
  };
  auto dma_v = [&](const __amdgpu_buffer_rsrc_t& rv, uint16_t* dst, int i) __attribute__((always_inline)) {
    const int blk = wave * VQPW + i;
    const int byte = blk * 1024 + lane * 16;
    const int r = byte / (DV * 2), p = (byte % (DV * 2)) / 16;
    int c = p ^ VShape::swz_v(r);
    if constexpr (DV != D) c %= D / 8;  // D=16: the padding chunks re-read their row's chunks
    lds_dma16<false>(rv, (uint8_t*)dst + blk * 1024, r * (int)vrow_bytes + c * 16);
  };
  auto load_k = [&](int n0, uint16_t* dst) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rk = k_rsrc(n0);
#pragma unroll
    for (int i = 0; i < QPW; ++i) dma_k(rk, dst, i);
  };
  auto load_v = [&](int n0, uint16_t* dst) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rv = v_rsrc(n0);
#pragma unroll
    for (int i = 0; i < VQPW; ++i) dma_v(rv, dst, i);
  };

  // ---- prologue, first half: K_0, V_0, K_1 and then Q go out before the rest of the set-up
  if (n_tiles > 0) {
    load_k(0, k_buf0);
    load_v(0, v_buf0);
    if (n_tiles > 1) load_k(BN, k_buf1);
  }
  __builtin_amdgcn_sched_barrier(0);
  load_q();
  __builtin_amdgcn_sched_barrier(0);

  // Per-lane LDS byte offsets of the MFMA operand reads.  Unsigned, so that the compiler may
  // fold the buffer bases and the per-slot constants into the ds_read offset field instead of
  // holding one address register per (buffer, slot) pair (16 VGPRs at D=128).
  // K: S^T A-operand, row kb*32 + j, logical chunk 2s + g.
  uint32_t koffs[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) koffs[s] = (uint32_t)(j * D + (((2 * s + g) ^ Shape::swz_k(j)) * 8)) * 2u;
  // V: ds_read_b64_tr_b16 sources, rows 8g + 4*hi + (i >> 2) of each 16-key step,
  // columns 32d + 16dh + 4(i & 3); the row term kb*32 + 16h is a constant offset.
  const int tr_i = lane & 15, tr_dh = (lane >> 4) & 1;
  uint32_t voffs[DB][2];
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int vr_row = 8 * g + 4 * hi + (tr_i >> 2);
      const int col = 32 * d + 16 * tr_dh + 4 * (tr_i & 3);
      voffs[d][hi] = (uint32_t)(vr_row * DV + (((col >> 3) ^ VShape::swz_v(vr_row)) * 8) + (col & 7)) * 2u;
    }
  }

  f32x16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16{};
  // running max m_run (log2 domain, scaled) and this lane's share of the row sum
  float m_run = NEG_INF, l_run = 0.f;
  f32x4 l_acc = f32x4{};  // MFMA_ROWSUM: every lane's registers hold its own row's full sum
  const u32x4 ones = rowsum_ones<E>(lane);
  // S^T of two consecutive tiles (the loop below is unrolled by 2)
  f32x16 s_a[KB], s_b[KB];

  // ---- building blocks ---------------------------------------------------------------
  auto qk = [&](const uint16_t* Ks, f32x16(&acc)[KB], int s) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      acc[kb] = mfma32<E>(ld16((const uint8_t*)Ks + (kb * 32 * D * 2 + koffs[s])), qf[s], acc[kb]);
  };
  // excluded scores of tile t (keys n0..n0+BN) -> -inf
  auto mask = [&](f32x16(&sc)[KB], int n0) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = n0 + kb * 32 + 16 * (r >> 3) + 8 * g + (r & 7);
        const bool ok = (n < khi) & ((a.causal == 0) | (n <= qlim));
        sc[kb][r] = ok ? sc[kb][r] : NEG_INF;
      }
    }
  };
  // row max of c*S over the tile (both lanes of the row agree)
  auto tile_max = [&](const f32x16(&sc)[KB]) __attribute__((always_inline)) {
    float mx = sc[0][0];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int r = (kb == 0 ? 1 : 0); r < 16; ++r) mx = vmax(mx, sc[kb][r]);
    }
    return max_xor32(mx * c);
  };
  // Lazy rescale: keep the running max unless some row of the wave grew by more
  // than 2^8; p = 2^(c*s - m_run) then stays <= 256, and O, l stay consistent
  // because both use the same m_run.
  auto update_max = [&](float mt) __attribute__((always_inline)) {
    const float m_new = vmax(m_run, mt);
    if (__builtin_amdgcn_ballot_w64(m_new > m_run + kRescaleLog2) != 0) {
      const float m_safe_new = (m_new == NEG_INF) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_safe_new);
      if constexpr (MFMA_ROWSUM) {
        l_acc *= alpha;
      } else {
        l_run *= alpha;
      }
#pragma unroll
      for (int d = 0; d < DB; ++d) oacc[d] *= alpha;
      m_run = m_new;
    }
  };
  // One pipelined iteration on tile t: S_{t+1} from K buffer Kn, P_t from cur,
  // O += V_t P_t from V buffer Vc, then the row max of S_{t+1}.  The max is taken
  // unmasked inside the main block and recomputed only when tile t+1 is masked
  // (or does not exist), so the common path is one basic block.
  // The DMA of the next tiles (K_{t+2} into kd, V_{t+1} into vd: buffers every wave has
  // finished reading) is issued one instruction per slot in the first NDMA slots, so every
  // load has the whole iteration to land before the end-of-iteration wait (measured against
  // one instruction every NM / NDMA slots: +1-3% causal N=4096, +2-5% at N=1024).
  auto body = [&](const uint16_t* Kn, const uint16_t* Vc, f32x16(&cur)[KB], f32x16(&nxt)[KB], int t,
                  const __amdgpu_buffer_rsrc_t& rk, uint16_t* kd, const __amdgpu_buffer_rsrc_t& rv, uint16_t* vd)
      __attribute__((always_inline)) {
    // MFMA slots m = 0 .. NQK-1: S_{t+1} (k-step m / KB, key block m % KB);
    // m = NQK .. NM-1: O += V_t P_t (key block, 16-key half, d block; d fastest).
    // The LDS operand of slot m is read PD slots ahead into a ring of registers,
    // so its latency (about two MFMAs) is hidden behind the MFMAs in between; a
    // sched_barrier after every slot keeps this order through scheduling.
    constexpr int NQK = KS * KB, NPV = KB * 2 * DB, NM = NQK + NPV, PD = 3;
    constexpr int NEXP = KB * 8;         // exp micro-steps (2 scores each) for S_t
    constexpr int NMAX = KB * 8;         // max3 steps for S_{t+1}
    // Where the vector work goes.  Exp step u (key block u / 8, 16-key half (u / 4) % 2) runs
    // in S slot u * NQK / ES for u < ES, else in one of the first PVW PV slots, always before
    // the first PV MFMA that reads its P half.  Max steps run in the PV slots from MAX0 on
    // (S_{t+1} is complete two slots after its last MFMA).  At D=128 the exponentials of the
    // second key block move into the first half of the PV slots and the max steps into the
    // second half, so every slot carries about the same vector work against its MFMA (measured
    // against all exponentials in the S slots: +0.5% causal N=4096, +2.1% non-causal N=4096,
    // +1.2% causal N=16384 at Hq=32 Hkv=8; N <= 2048 unchanged).
    constexpr int ES = D == 128 ? NEXP / 2 : NEXP;
    constexpr int PVW = NPV / 2;
    constexpr int MAX0 = D == 128 ? NPV / 2 : 2;
    static_assert(ES % NQK == 0 || NQK % ES == 0, "exp steps must spread evenly over the S slots");
    auto exp_slot = [](int u) constexpr {
      return u < ES ? u * NQK / ES : NQK + (u - ES) * PVW / (NEXP > ES ? NEXP - ES : 1);
    };
    // the first PV slot that reads the P half of exp step u
    auto exp_deadline = [](int u) constexpr { return NQK + ((u / 8) * 2 + (u / 4) % 2) * DB; };
    constexpr int NDMA = QPW + VQPW;
    static_assert(NDMA <= NM, "one DMA instruction per slot");
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) nxt[kb] = f32x16{};
    const float m_safe = (m_run == NEG_INF) ? 0.f : m_run;
    u32x4 pf[KB][2];
    u32x4 opnd[PD + 1];
    float rs = 0.f;
    float mx = NEG_INF;

    auto read = [&](int m) __attribute__((always_inline)) {
      if (m < NQK) {
        const int s = m / KB, kb = m % KB;
        opnd[m % (PD + 1)] = ld16((const uint8_t*)Kn + (kb * 32 * D * 2 + koffs[s]));
      } else {
        const int i = m - NQK, kb = i / (2 * DB), h = (i / DB) % 2, d = i % DB;
        const uint8_t* vp = (const uint8_t*)Vc + (kb * 32 + 16 * h) * DV * 2;
        const u32x2 lo = lds_read_tr16((const uint16_t*)(vp + voffs[d][0]));
        const u32x2 hi = lds_read_tr16((const uint16_t*)(vp + voffs[d][1]));
        opnd[m % (PD + 1)] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    };
    // exp micro-step u: scores 2e and 2e+1 of chunk (kb, h) of S_t
    auto exp_step = [&](int u) __attribute__((always_inline)) {
      const int kb = u / 8, h = (u / 4) % 2, e = u % 4;
      const float p0 = fast_exp2(__builtin_fmaf(cur[kb][8 * h + 2 * e], c, -m_safe));
      const float p1 = fast_exp2(__builtin_fmaf(cur[kb][8 * h + 2 * e + 1], c, -m_safe));
      const uint32_t pk = pack2<E>(p0, p1);
      pf[kb][h][e] = pk;
      // the row sum of the rounded P that the MFMA consumes (so O/l is a convex combination)
      if constexpr (!MFMA_ROWSUM) rs = sum2<E>(pk, rs);
    };
    // max step v: scores 2v and 2v+1 of S_{t+1}
    auto max_step = [&](int v) __attribute__((always_inline)) {
      const int kb = v / 8, r = 2 * (v % 8);
      mx = vmax(vmax(mx, nxt[kb][r]), nxt[kb][r + 1]);  // one v_maximum3 per two scores
    };

    // (static_for: every slot index is a compile-time constant, so the operand ring, the
    // accumulator indices and the LDS offsets resolve without relying on loop unrolling)
    static_for<0, PD>([&](auto mc) __attribute__((always_inline)) { read(decltype(mc)::value); });
    static_for<0, NM>([&](auto mc) __attribute__((always_inline)) {
      constexpr int m = decltype(mc)::value;
      if constexpr (m + PD < NM) read(m + PD);
      if constexpr (m < NDMA) {
        if constexpr (m < QPW) {
          dma_k(rk, kd, m);
        } else {
          dma_v(rv, vd, m - QPW);
        }
      }
      const u32x4 op = opnd[m % (PD + 1)];
      if constexpr (m < NQK) {
        constexpr int s = m / KB, kb = m % KB;
        nxt[kb] = mfma32<E>(op, qf[s], nxt[kb]);
        static_for<0, NEXP>([&](auto uc) __attribute__((always_inline)) {
          constexpr int u = decltype(uc)::value;
          static_assert(exp_slot(u) < exp_deadline(u), "P must be complete before its PV MFMA");
          if constexpr (exp_slot(u) == m) exp_step(u);
        });
      } else {
        constexpr int i = m - NQK, kb = i / (2 * DB), h = (i / DB) % 2, d = i % DB;
        oacc[d] = mfma32<E>(op, pf[kb][h], oacc[d]);
        if constexpr (MFMA_ROWSUM) {
          if constexpr (d == 0) l_acc = mfma16<E>(ones, pf[kb][h], l_acc);  // row sums of 16 keys of P_t
        }
        static_for<0, NEXP>([&](auto uc) __attribute__((always_inline)) {
          constexpr int u = decltype(uc)::value;
          if constexpr (exp_slot(u) == m) exp_step(u);
        });
        if constexpr (i >= MAX0) {
          constexpr int v0 = (i - MAX0) * NMAX / (NPV - MAX0), v1 = (i - MAX0 + 1) * NMAX / (NPV - MAX0);
          static_for<v0, v1>([&](auto vc) __attribute__((always_inline)) { max_step(decltype(vc)::value); });
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    l_run += rs;
    float mt = max_xor32(mx * c);
    if (t + 1 >= n_fast) {
      const int n1 = (t + 1) * BN;
      if (t + 1 < n_tiles) {
        if (n1 + BN > mask_from) {
          // an empty volatile asm cannot be speculated: without it the compiler
          // if-converts this rare branch and masks every tile in the hot block
          // (measured: ~150 extra VALU/SALU instructions per tile)
          __asm__ volatile("");
          mask(nxt, n1);
          mt = tile_max(nxt);
        }
      } else {
        mt = NEG_INF;  // past the last tile: nxt holds stale LDS data and is discarded
      }
    }
    update_max(mt);
  };

  // ---- prologue: K_0, V_0, K_1 in flight; S_0 and its max ------------------------------
  {
    const uint32_t keep = row_ok ? 0xffffffffu : 0u;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = (qf[s] ^ qsign) & keep;
  }
  if (n_tiles > 0) {
    lds_dma_wait();
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) s_a[kb] = f32x16{};
#pragma unroll
    for (int s = 0; s < KS; ++s) qk(k_buf0, s_a, s);
    if (BN > mask_from) mask(s_a, 0);
    update_max(tile_max(s_a));
    __syncthreads();  // every wave has read K_0: its buffer takes K_2
  }

  // ---- main loop, unrolled by 2 so that every buffer is named at compile time --------
  auto step = [&](auto stage_tag, int t) __attribute__((always_inline)) {
    constexpr int ST = decltype(stage_tag)::value;
    uint16_t* k_this = ST == 0 ? k_buf0 : k_buf1;  // held K_t (read already), takes K_{t+2}
    uint16_t* k_next = ST == 0 ? k_buf1 : k_buf0;  // holds K_{t+1}
    uint16_t* v_this = ST == 0 ? v_buf0 : v_buf1;  // holds V_t
    uint16_t* v_next = ST == 0 ? v_buf1 : v_buf0;  // takes V_{t+1}
    auto& cur = ST == 0 ? s_a : s_b;
    auto& nxt = ST == 0 ? s_b : s_a;
    // K_{t+2} and V_{t+1} (zero-length descriptors past the last tile)
    if (NW == 4 || t < wave_tiles) {
      body(k_next, v_this, cur, nxt, t, k_rsrc((t + 2) * BN), k_this, v_rsrc((t + 1) * BN), v_next);
    } else {
      const __amdgpu_buffer_rsrc_t rk = k_rsrc((t + 2) * BN), rv = v_rsrc((t + 1) * BN);
#pragma unroll
      for (int i = 0; i < QPW; ++i) dma_k(rk, k_this, i);
#pragma unroll
      for (int i = 0; i < VQPW; ++i) dma_v(rv, v_next, i);
    }
    lds_dma_wait();
    __syncthreads();
  };
  for (int t = 0; t < n_tiles; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < n_tiles) step(std::integral_constant<int, 1>{}, t + 1);
  }

  // ---- epilogue ------------------------------------------------------------------------
  if (!wave_active) return;
  // each lane summed its 16 of the row's keys per tile (or holds the full sum, MFMA_ROWSUM)
  const float l_tot = MFMA_ROWSUM ? l_acc[0] : sum_xor32(l_run);
  // Rows that saw no key have l == 0 and emit zeros (triton_fwd.py:163-165).
  const float l_safe = (l_tot == 0.f) ? 1.f : l_tot;
  const float inv = 1.f / l_safe;
  // O is staged through LDS, row-major with 16-byte chunks XOR-swizzled by row, and written
  // back in whole rows: a lane of the O^T fragment holds 4 values of each of 16 chunks of one
  // row, so storing from the fragment sends each instruction to 32 rows (32 partial cache
  // lines); from LDS, 16 consecutive lanes write one row's 256 bytes (D=128).  Every wave has
  // passed the last tile's barrier and its DMA has landed, so the K/V buffers are free; each
  // wave takes its own 32*D-element region of them.
  {
    constexpr int NCH = D / 8;                       // 16-byte chunks per row
    constexpr int SWZ = NCH < 16 ? NCH - 1 : 15;     // chunk swizzle by row
    constexpr int REG = 32 * D;                      // elements per wave
    constexpr int PER_BUF = TILE / REG;              // wave regions per buffer
    static_assert(PER_BUF >= 1 && VTILE >= TILE && NW <= 4 * PER_BUF, "O staging must fit the K/V buffers");
    const int bi = wave / PER_BUF;
    uint16_t* stage = (bi == 0 ? k_buf0 : bi == 1 ? k_buf1 : bi == 2 ? v_buf0 : v_buf1) + (wave % PER_BUF) * REG;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        if (d * 32 + 8 * rq >= D) continue;  // D=16: O^T rows 16..31 are padding
        const int c = 4 * d + rq;            // chunk of d values d*32 + 8*rq .. +7; this lane holds half g
        *reinterpret_cast<u32x2*>(stage + j * D + ((c ^ (j & SWZ)) * 8) + 4 * g) =
            u32x2{pack2<E>(oacc[d][4 * rq] * inv, oacc[d][4 * rq + 1] * inv),
                  pack2<E>(oacc[d][4 * rq + 2] * inv, oacc[d][4 * rq + 3] * inv)};
      }
    }
    constexpr int RPI = 64 / NCH;  // rows per 64-lane read
    const int cc = lane % NCH;
    uint16_t* obase = (uint16_t*)a.o + (int64_t)b * a.sob + (int64_t)hq * a.soh + (qtok0 + wr0) * a.son;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = i * RPI + lane / NCH;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * D + ((cc ^ (r & SWZ)) * 8));
      if (wr0 + r < seq_q) {
        uint16_t* dst = obase + (int64_t)r * a.son + cc * 8;
        if (a.o16) {
          st16(dst, v);
        } else {
          st8(dst, u32x2{v[0], v[1]});
          st8(dst + 4, u32x2{v[2], v[3]});
        }
      }
    }
  }
  if (row_ok && a.lse != nullptr && g == 0) {
    // natural-log LSE (triton_fwd.py:169-172)
    a.lse[(int64_t)b * a.slb + (int64_t)hq * a.slh + (qtok0 + qi)] = (m_run + __log2f(l_safe)) * kLn2;
  }
}

template <int D, class E, int NW>
static hipError_t launch_fwd(const TileArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_kernel<D, E, NW>), dim3((unsigned)a.total), dim3(NW * 64), 0, stream, a);
  return hipGetLastError();
}

fa_status run_fwd(const fa_fwd_params& p, bool varlen, hipStream_t stream, const char** err) {
  const bool mfma = (p.dtype == FA_DTYPE_BF16 || p.dtype == FA_DTYPE_F16) &&
                    (p.head_dim == 16 || p.head_dim == 32 || p.head_dim == 64 || p.head_dim == 128 ||
                     p.head_dim == 256);
  if (p.dtype == FA_DTYPE_F32 && p.head_dim >= 32)
    return run_fwd_f32(p, varlen, stream, err);
  if (!mfma) return run_fwd_generic(p, varlen, stream, err);
  TileArgs a = common_args(p);
  a.o = p.o;
  a.sob = p.o_stride_b;
  a.soh = p.o_stride_h;
  a.son = p.o_stride_n;
  a.o16 = (reinterpret_cast<uintptr_t>(p.o) % 16 == 0 && p.o_stride_h % 8 == 0 && p.o_stride_n % 8 == 0 &&
           (varlen || p.o_stride_b % 8 == 0)) ? 1 : 0;
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
  // Dense D=128 with at least 4096 queries (2048 without the causal mask) runs 8 waves (256
  // queries) per workgroup: each K/V tile feeds twice the rows, halving the DMA per MFMA
  // (measured over 4 waves, Hq=32 Hkv=8: +1% causal at N=4096, +2% at 8192 and 16384, +1.7%
  // non-causal at 2048).  Shorter sequences keep 4 (more, shorter workgroups whose start
  // overlaps the other workgroup on the CU: 8 waves lose 5% causal at N=1024, 2.5% at 2048,
  // 0.7% non-causal at 1024).  D=64 keeps 4 (-3% with 8) and D=256 runs one wave per SIMD.
  // Varlen applies the same rule to its longest sequence (max_seqlen_q): a causal batch of 16
  // sequences of 0-4073 tokens keeps 4 waves, and 8 from 2048 measured 2-5% slower on it (its
  // short sequences leave more of a 256-query block empty).  A wave computes the same tiles
  // in the same order with 4 or 8 waves per workgroup, so the result does not depend on the
  // choice.
  const int nw = (p.head_dim == 128 && a.nq >= (p.causal ? 4096 : 2048)) ? 8 : 4;
  a.n_rowblk = (a.nq + nw * 32 - 1) / (nw * 32);
  const int64_t kv_groups = (int64_t)p.batch * p.heads_kv;
  // varlen: the (sequence, kv-head) groups are padded to a multiple of the 8 XCDs
  const int64_t groups = varlen ? (kv_groups + 7) / 8 * 8 : kv_groups;
  const int64_t total = groups * a.group * a.n_rowblk;
  if (total > INT32_MAX) {
    *err = "grid too large";
    return FA_ERR_UNSUPPORTED;
  }
  a.total = (int32_t)total;
  a.kv_groups = (int32_t)kv_groups;
  // a unit never holds more than the (batch, q-head) pairs there are, which keeps u_items <= total
  a.u_heads = (int32_t)std::min<int64_t>(prefill_unit_heads(a.nk, p.head_dim, a.group), kv_groups * a.group);
  a.u_items = a.u_heads * a.n_rowblk;
  a.n_split = 1;
  a.split_len = 0;
  hipError_t e = hipErrorInvalidValue;
  const bool bf = p.dtype == FA_DTYPE_BF16;
  if (p.head_dim == 128) {
    if (nw == 8) {
      e = bf ? launch_fwd<128, BF16, 8>(a, stream) : launch_fwd<128, F16, 8>(a, stream);
    } else {
      e = bf ? launch_fwd<128, BF16, 4>(a, stream) : launch_fwd<128, F16, 4>(a, stream);
    }
  } else if (p.head_dim == 64) {
    e = bf ? launch_fwd<64, BF16, 4>(a, stream) : launch_fwd<64, F16, 4>(a, stream);
  } else if (p.head_dim == 32) {
    e = bf ? launch_fwd<32, BF16, 4>(a, stream) : launch_fwd<32, F16, 4>(a, stream);
  } else if (p.head_dim == 16) {
    e = bf ? launch_fwd<16, BF16, 4>(a, stream) : launch_fwd<16, F16, 4>(a, stream);
  } else if (p.head_dim == 256) {
    e = bf ? launch_fwd<256, BF16, 4>(a, stream) : launch_fwd<256, F16, 4>(a, stream);
  }
  return hip_status(e, err);
}

}  // namespace fa
