// One range of work units of the decode-regime HEX expert GEMM (the per-projection kernels of
// hex_moe.hip).
//
//  * Units of work are (expert block of the slot plan, 256-row tile, 256-input unit). A launch
//    cuts them into G contiguous ranges [U g / G, U (g + 1) / G), one per workgroup turn, so
//    every range streams the same number of units and consecutive units mostly share an expert
//    and its LDS tables. An item (block, row tile) split between ranges is finished by the last
//    of them to arrive, which adds the others' partial sums (left in a workspace with
//    device-coherent stores) in range order, so the result does not depend on timing.
//  * Each wave owns 16 rows of the tile. Each lane streams the packed words of one whole
//    32-input block per row per step with one 128-bit load (4-bit; three dwords at 3-bit):
//    row = lane % 16, block 4 s + lane / 16. Loads run P units ahead of the math in registers,
//    across item boundaries, so HBM sees a steady stream of requests.
//  * A trip's activation tiles (16 slots x 128 inputs per 16-slot subtile and step) are fetched
//    once per workgroup, a dword per lane, and passed through a two-stage LDS ring to all waves.
//  * A 4x4 transpose across the wave's rows (permlane swaps) gives each lane the 8 codes the
//    16x16x32 MFMA wants from it, with all 32 inputs of one MFMA inside one HEX block, so every
//    MFMA partial carries exactly one fp8 block scale.
//  * Codes resolve through a pair table in LDS: entry p = (level[p & (L-1)], level[p >> bits])
//    rounded to the activation dtype and packed, so one ds_read_b32 yields two operands. The
//    table has one copy per lane in its own bank (32 copies each for gate and up, 64 for down);
//    the read address is (pair << 8) | lane copy offset, one v_perm_b32 at 4 bits. It is
//    rebuilt only when the expert changes.
//  * The fp32 partial of each block times its fp8 scale is added to the accumulator; the expert
//    scale, SiLU * up, and the top-k weight are applied in the epilogue, in the reference's order
//    (runtime/blackhole_runtime/hex_moe.py:109-151).
// Weights therefore enter the matrix cores as round(level) and the block scale is applied to
// the float32 block partial, where the reference rounds level * fp8 to the activation dtype.
#pragma once

#include <type_traits>

#include "hex_fused.h"

namespace bh {

// One unit's loads of one wave: two 128-input steps.
template <int BITS, int NM, int SB, bool KF>
struct Stage {
  using W = typename std::conditional<BITS == 4, u32x4, u32x3>::type;
  W w[NM][2];            // per step, the lane's 32-input block (4-bit: 4 words; 3-bit: 3)
  // fp8 block scales of the row: whole units read them in one load (8 bytes at B = 32, 2 at
  // B = 128); the tail variant reads them byte by byte
  typename std::conditional<SB == 1, u32x2, uint32_t>::type scw[NM];
  uint32_t scb[NM][KF ? 1 : (SB == 1 ? 8 : 2)];
};

// Buffer descriptors of the weight stream's current item. Each spans one expert's matrix, so
// loads past its end return zero instead of faulting; rows past the matrix read out of range
// (nothing fetched) and are never stored.
template <int NM>
struct ItemRes {
  __amdgpu_buffer_rsrc_t rw[NM];   // packed index words of the item's expert
  __amdgpu_buffer_rsrc_t rb[NM];   // its fp8 block scales
  uint32_t vw[NM], vb[NM];         // lane offsets: row n, block lane / 16 of the unit
};

// The hot loop keeps every load unconditional and in a fixed order, so the compiler's waits
// for them stay partial (vmcnt(N), not 0).

// Expert blocks a range may touch (their experts and slot rows are staged in LDS); launches
// size their ranges so that none needs more. At 16-slot blocks; 64 / MT in general.
constexpr int kMaxBlk16 = 64;
constexpr int kMaxExperts = 1024;        // global expert ids the tier lookup may take

constexpr int kThreads = 1024;           // 16 waves, one workgroup per compute unit
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 16 * kWaves;       // output rows of one work item: 16 per wave
constexpr int kMinUnits = 2;             // units per workgroup below which the grid shrinks
                                         // (1 measured slower: config 2 at 1 token, 44.1 against
                                         // 40.5 us, the second unit's loads no longer hidden)

// Units per trip P: the weight loads of P units are in flight per wave ahead of the math, and
// the activation tiles of the next P units are fetched one trip ahead; one workgroup barrier
// per trip publishes them. (Four units per trip for the 16-slot down kernel measured slower at
// config 2, T=16: 66.9 against 64.6 us per layer; its larger first trip delays the prologue.)
template <int MT, bool GLU>
constexpr int trip() { return GLU ? (MT == 1 ? 2 : 1) : (MT == 4 ? 1 : 2); }

// Position of a unit: block (relative to the range's first), row tile, unit within the item.
struct Pos {
  int pm, pn, s;
};

// Partial sums of one wave's 16 x BM tile, [mt][m][lane][4] floats.
template <int MT, int NM>
constexpr int part_floats() { return MT * NM * kWave * 4; }

// Range g of G holding unit u of U.
// (32-bit arithmetic throughout: the host refuses launches whose U * G does not fit in 31 bits,
// and 64-bit divisions would cost hundreds of scalar instructions each before the first load.)
__device__ __forceinline__ int owner(uint32_t u, uint32_t U, uint32_t G) {
  return (int)(((u + 1) * G + U - 1) / U - 1);
}

// The cut of a launch's units into ranges, for `used` plan blocks over an N x K projection
// and `grid` workgroups. Whole items when that balances well enough: with q = ceil(items / grid)
// items per range, q = 1 and at least half as many items as workgroups, or q > 1 and the ranges
// at least 3/4 full on average; then Q = q and range g is items [g q, (g + 1) q), so no item is
// split and no partial sums are exchanged. Otherwise (Q = 0) the units are spread evenly over
// min(grid, U) ranges, splitting items.
struct Ranges {
  uint32_t U, G, Q;
};
__host__ __device__ __forceinline__ Ranges moe_ranges(uint32_t used, int N, int K, uint32_t grid) {
  const uint32_t nrt = (uint32_t)(N + kRows - 1) / kRows;
  const uint32_t nun = ((uint32_t)K / kHexBlock + 7) / 8;
  const uint32_t items = used * nrt;
  Ranges r;
  r.U = items * nun;
  const uint32_t q = (items + grid - 1) / grid;
  const bool whole = items > 0 && (q == 1 ? 2 * items >= grid : 4 * items >= 3 * q * grid);
  r.Q = whole ? q : 0;
  r.G = whole ? (items + q - 1) / q : (grid < r.U ? grid : r.U);
  return r;
}

// The most slots a launch may sort in its own workgroups (one per thread) instead of taking a
// plan from the align kernel.
constexpr int kPlanMaxSlots = kThreads;

// LDS of the in-kernel slot plan (it lives where the activation ring will, before the ring's
// first use): slots of each (wave, expert), as bytes (a wave holds at most 64 slots), the
// expert's first block, and the scan's wave sums.
struct PlanLds {
  uint8_t wcnt[kWaves][kMaxExperts];
  int first[kMaxExperts];
  int wsum[kWaves];
  int used;
};

// LDS of one range. The pair tables come first: their base stays inside the ds offset field.
template <int BITS, bool GLU, int MT>
struct alignas(16) MoeSmem {
  static constexpr int L = 1 << BITS, NPAIR = 1 << (2 * BITS), NM = GLU ? 2 : 1, BM = 16 * MT;
  static constexpr int P = trip<MT, GLU>(), MAXBLK = kMaxBlk16 / MT, TILE = MT * 1024;
  uint32_t tab[NPAIR * 64];
  union {
    uint32_t ring[2][P * 2 * TILE];      // a trip's activation tiles, two trips
    PlanLds plan;                        // the in-kernel slot plan (prologue only)
  };
  int lut[kMaxExperts];                  // the tier lookup
  int slots[MAXBLK * BM];                // slot rows of the range's blocks
  float slot_w[GLU ? 1 : MAXBLK * BM];   // their top-k weights (down)
  int blk_g[MAXBLK];                     // global expert of each block
  int blk_e[MAXBLK];                     // its tier-local expert, -1 for none
  float blk_es[MAXBLK][NM];              // expert scales
  uint16_t blk_lv[MAXBLK][NM][L];        // levels in the activation dtype
  int split_last[2];                     // this workgroup finishes split item k
};

template <int BITS, int ADT, bool GLU, int MT, int SB, bool KF>
__device__ __forceinline__ void moe_range(const MoeArgs& a, MoeSmem<BITS, GLU, MT>& sm, const uint32_t g, const int tid) {
  static_assert(sizeof(PlanLds) <= sizeof(sm.ring), "the plan's LDS must fit in the ring");
  constexpr int L = 1 << BITS;
  constexpr int NPAIR = 1 << (2 * BITS);
  constexpr int NM = GLU ? 2 : 1;
  constexpr int BM = 16 * MT;
  constexpr int P = trip<MT, GLU>();
  constexpr int MAXBLK = kMaxBlk16 / MT;
  constexpr int PF = part_floats<MT, NM>();
  constexpr int TILE = MT * 1024;               // dwords of one step's activation tile
  // Everything a unit needs besides its streamed weights and activations is staged in LDS at
  // the start. The activation tiles of a trip (P units x 2 steps) go through a two-trip ring:
  // fetched once per workgroup, a dword per lane per tile, and read by all 16 waves.
  auto& tab = sm.tab;
  auto& ring = sm.ring;
  auto& lut = sm.lut;
  auto& slots = sm.slots;
  auto& slot_w = sm.slot_w;
  auto& blk_g = sm.blk_g;
  auto& blk_e = sm.blk_e;
  auto& blk_es = sm.blk_es;
  auto& blk_lv = sm.blk_lv;
  auto& split_last = sm.split_last;

  const int lane = tid & 63, ln = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: units and row tiles stay scalar
  const int nrt = (a.N + kRows - 1) / kRows;
  const int nb32 = a.K / kHexBlock;
  const int nun = (nb32 + 7) / 8;                              // units per item

  // ---- the slot plan from the routing ids (a.ids set): every workgroup sorts the slots by
  // expert in LDS, with the align kernel's algorithm and result (a stable counting sort, each
  // expert's run padded to whole blocks), and keeps the part its range needs. A thread per
  // slot: a wave finds the lanes holding its key by ballots; the key's lowest lane records the
  // wave's count; one pass over the waves gives each expert's total, a workgroup scan its first
  // block, and each slot's row is that block's first row + the expert's slots in earlier waves
  // + its rank among the wave's lanes of the same key.
  uint32_t used;
  int my_row = -1, my_nb = 0, my_first = 0;     // this thread's slot row; its expert's blocks
  if (a.ids) {
    PlanLds& ps = sm.plan;
    const int S = (int)a.num_slots, E = a.n_experts;
    const int nw = (S + kWave - 1) / kWave;
    int64_t id = -1;
    if (tid < S) id = a.ids_i64 ? reinterpret_cast<const int64_t*>(a.ids)[tid] : reinterpret_cast<const int32_t*>(a.ids)[tid];
    if (tid < E) lut[tid] = a.lookup[tid];
    for (int i = tid; i < nw * (kMaxExperts / 4); i += kThreads) reinterpret_cast<uint32_t*>(ps.wcnt)[i] = 0u;
    // the staged plan's rows start empty (they lie outside the plan's LDS)
    for (int b = tid; b < MAXBLK; b += kThreads) blk_g[b] = -1;
    for (int r = tid; r < MAXBLK * BM; r += kThreads) slots[r] = (int)a.num_slots;
    __syncthreads();
    const int key = (id >= 0 && id < E && lut[id] >= 0) ? (int)id : E;
    int nbits = 1;
    while ((1 << nbits) <= E) ++nbits;        // keys in [0, E] (E: not placed)
    const uint64_t same = match_key(key, nbits);
    const int rank = __popcll(same & (lane ? (~0ull >> (64 - lane)) : 0ull));
    if (key < E && rank == 0) ps.wcnt[wave][key] = (uint8_t)__popcll(same);
    __syncthreads();
    int c = 0, before = 0;
    if (tid < E)
      for (int v = 0; v < nw; ++v) c += ps.wcnt[v][tid];
    if (key < E)
      for (int v = 0; v < wave; ++v) before += ps.wcnt[v][key];
    my_nb = (c + BM - 1) / BM;
    const int incl = block_incl_scan(my_nb, ps.wsum);   // (its barriers order the reads above)
    my_first = incl - my_nb;
    if (tid < E) ps.first[tid] = my_first;
    if (tid == kThreads - 1) ps.used = incl;
    __syncthreads();
    used = ps.used;
    if (key < E) my_row = ps.first[key] * BM + before + rank;
  } else {
    used = a.npp[0] / BM;
  }
  const Ranges rg = moe_ranges(used, a.N, a.K, gridDim.x);
  if (g >= rg.G) return;                                       // (uniform: no work for this workgroup)

  // ---- this range of units over the used blocks
  const uint32_t U = rg.U, G = rg.G;
  const uint32_t ub = rg.Q ? g * rg.Q * nun : U * g / G;
  const uint32_t ue = rg.Q ? min(U, (g + 1) * rg.Q * nun) : U * (g + 1) / G;
  const int n = (int)(ue - ub);
  const uint32_t item0 = ub / nun, item1 = (ue - 1) / nun;
  const uint32_t pm0 = item0 / nrt;
  const int nblk = min((int)(item1 / nrt - pm0 + 1), MAXBLK);

  // ---- stage the plan: tier lookup, block experts, slot rows (S for padding)
  if (a.ids) {
    // thread e holds expert e's run, blocks [my_first, my_first + my_nb): those in this range
    const int j1 = min(my_first + my_nb, (int)pm0 + nblk);
    for (int j = max(my_first, (int)pm0); j < j1; ++j) blk_g[j - pm0] = tid;
    if (my_row >= 0) {
      const int r = my_row - (int)pm0 * BM;
      if (r >= 0 && r < nblk * BM) slots[r] = tid;
    }
  } else {
    for (int i = tid; i < a.n_experts; i += kThreads) lut[i] = a.lookup[i];
    for (int b = tid; b < MAXBLK; b += kThreads) blk_g[b] = b < nblk ? a.eid[pm0 + b] : -1;
    for (int r = tid; r < MAXBLK * BM; r += kThreads)
      slots[r] = r < nblk * BM ? a.sid[pm0 * BM + r] : (int)a.num_slots;
  }
  __syncthreads();
  auto expert_of = [&](int b) {      // tier-local expert of block b, -1 for none
    const int eg = blk_g[b];
    return (eg >= 0 && eg < a.n_experts) ? lut[eg] : -1;
  };

  uint32_t cb[NM];
  if constexpr (GLU) {
    cb[0] = (lane & 31u) * 4u;
    cb[NM - 1] = 128u + (lane & 31u) * 4u;
  } else {
    cb[0] = lane * 4u;
  }
  auto advance = [&](Pos& p) {
    if (++p.s == nun) {
      p.s = 0;
      if (++p.pn == nrt) {
        p.pn = 0;
        ++p.pm;
      }
    }
  };

  // ---- weight stream: buffer loads, per-item descriptors
  ItemRes<NM> R;
  constexpr int BLKB = BITS * 4;               // bytes of one 32-input block of one row
  constexpr int USTEP = 8 * BLKB;              // bytes of one unit of one row
  auto setup = [&](const Pos& p) {
    const int b = min(p.pm, MAXBLK - 1);
    const int e = __builtin_amdgcn_readfirstlane(expert_of(b));   // uniform: keeps descriptors scalar
    const int nrow = p.pn * kRows + wave * 16 + ln;
    const bool rv = e >= 0 && nrow < a.N;            // rows past the matrix fetch nothing
    const int64_t ee = e >= 0 ? e : 0;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const bh_hex_proj& w = m == 0 ? a.w0 : a.w1;
      R.rw[m] = buffer_rsrc(w.idx + ee * w.s_ie, (int64_t)a.N * w.s_in * 4);
      R.rb[m] = buffer_rsrc(w.block_scale + ee * w.s_be, (int64_t)a.N * w.s_bn);
      R.vw[m] = rv ? (uint32_t)(nrow * w.s_in * 4) + lg * BLKB : kOOR;
      R.vb[m] = rv ? (uint32_t)(nrow * w.s_bn) : kOOR;
    }
  };
  // loads of unit s of the current descriptors; dummy units (past the range) read out of range.
  // per matrix: the two steps' blocks, then the unit's scales
  // The whole byte offset goes in the range-checked VGPR offset (soffset 0): dummy units and
  // invalid rows sit past every resource.
  auto load = [&](int s_, bool real, Stage<BITS, NM, SB, KF>& st) {
    const int s = __builtin_amdgcn_readfirstlane(real ? s_ : 0);
    const uint32_t ws = real ? (uint32_t)(s * USTEP) : kOOR;
    const uint32_t bs = real ? (uint32_t)((SB == 1 ? 8 : 2) * s) : kOOR;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const uint32_t vw = R.vw[m] + ws, vb = R.vb[m] + bs;
      if constexpr (BITS == 4) {
        ld_x4<0>(st.w[m][0], R.rw[m], vw);
        ld_x4<4 * BLKB>(st.w[m][1], R.rw[m], vw);
      } else {
        ld_x3<0>(st.w[m][0], R.rw[m], vw);
        ld_x3<4 * BLKB>(st.w[m][1], R.rw[m], vw);
      }
      if constexpr (KF) {
        if constexpr (SB == 1) ld_x2<0>(st.scw[m], R.rb[m], vb);
        else ld_u16<0>(st.scw[m], R.rb[m], vb);
      } else {
        ld_u8<0>(st.scb[m][0], R.rb[m], vb);
        ld_u8<1>(st.scb[m][1], R.rb[m], vb);
        if constexpr (SB == 1) {
          ld_u8<2>(st.scb[m][2], R.rb[m], vb);
          ld_u8<3>(st.scb[m][3], R.rb[m], vb);
          ld_u8<4>(st.scb[m][4], R.rb[m], vb);
          ld_u8<5>(st.scb[m][5], R.rb[m], vb);
          ld_u8<6>(st.scb[m][6], R.rb[m], vb);
          ld_u8<7>(st.scb[m][7], R.rb[m], vb);
        }
      }
    }
  };

  // ---- activation stream: the tiles of the next trip, one dword per lane per (unit, step, subtile)
  const int x_rows = (int)(((uint32_t)a.num_slots + (uint32_t)a.a_div - 1) / (uint32_t)a.a_div);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (int64_t)x_rows * a.s_xm * 2);
  // lane dword of a step's tile: wave w, lane l -> slot l / 4 of the subtile, inputs
  // 32 (w / 4) + 8 (w % 4) + 2 (l % 4) of the step (the fragment layout the MFMA reads)
  const int xcol = (wave >> 2) * 64 + (wave & 3) * 16 + (lane & 3) * 4;
  uint32_t vx[MT];
  int ax_b = -1;
  auto act_rows = [&](int b) {
    const int e = expert_of(b);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {            // padding slots fetch nothing
      const int slot = slots[b * BM + mt * 16 + (lane >> 2)];
      vx[mt] = (e >= 0 && slot < a.num_slots) ? (uint32_t)((int64_t)(slot / a.a_div) * a.s_xm * 2) + xcol : kOOR;
    }
  };
  uint32_t ax[P][2][MT];
  Pos ap{0, (int)(item0 - pm0 * nrt), (int)(ub - item0 * nun)};
  int ja = 0;
  auto act_trip = [&]() {                        // loads of the next P units' tiles
    uint32_t xs[P][2], vxd[P][MT];
#pragma unroll
    for (int d = 0; d < P; ++d) {
      const bool real = ja < n;
      const int b = min(ap.pm, MAXBLK - 1);
      if (real && b != ax_b) {
        act_rows(b);
        ax_b = b;
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) vxd[d][mt] = vx[mt];
#pragma unroll
      for (int h = 0; h < 2; ++h) xs[d][h] = (uint32_t)__builtin_amdgcn_readfirstlane((int)(real ? (uint32_t)(2 * ap.s + h) * 256 : kOOR));
      advance(ap);
      ++ja;
    }
#pragma unroll
    for (int d = 0; d < P; ++d)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) ax[d][h][mt] = __builtin_amdgcn_raw_buffer_load_b32(rx, voff(vxd[d][mt] + xs[d][h]), 0, 0);
  };

  // ---- compute stream
  f32x4 acc[MT][NM];
  // One unit = 8 MFMA k-slices (2 steps x 4 blocks). The table reads and the activation fragment
  // of slice k + 1 are issued before the MFMAs of slice k, so LDS latency hides behind them.
  auto compute = [&](int s, const Stage<BITS, NM, SB, KF>& st, const uint32_t* tiles) {
    uint32_t r[2][NM][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int m = 0; m < NM; ++m) fields<BITS>(st.w[m][h], r[h][m]);   // r[h][m][q]: block 8 s + 4 h + q
    const int nk = KF ? 8 : min(8, nb32 - 8 * s);   // valid k-slices of this unit
    u32x4 bq[2][NM], av[2][MT];
    auto fetch = [&](int k, int slot) {
#pragma unroll
      for (int m = 0; m < NM; ++m) bq[slot][m] = lookup8<BITS>(r[k >> 2][m][k & 3], cb[m], tab);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        av[slot][mt] = *reinterpret_cast<const u32x4*>(tiles + (k >> 2) * TILE + mt * 1024 + (k & 3) * 256 + lane * 4);
    };
    f32x4 part[MT][NM];
    float sf[NM][4];                 // B = 32: the step's 4 block scales
    fetch(0, 0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int h = k >> 2, q = k & 3;
      if (q == 0) {
        if constexpr (SB == 1) {
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            uint32_t w4;
            if constexpr (KF) w4 = st.scw[m][h];
            else w4 = st.scb[m][4 * h] | (st.scb[m][4 * h + 1] << 8) | (st.scb[m][4 * h + 2] << 16) | (st.scb[m][4 * h + 3] << 24);
            fp8x4(w4, sf[m]);
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int m = 0; m < NM; ++m) part[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      if (k + 1 < 8 && (KF || k + 1 < nk)) fetch(k + 1, (k + 1) & 1);
      if (KF || k < nk) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            if constexpr (SB == 1) {
              const f32x4 pr = mfma16x16x32<ADT>(av[k & 1][mt], bq[k & 1][m], f32x4{0.f, 0.f, 0.f, 0.f});
              acc[mt][m] += pr * sf[m][q];
            } else {
              part[mt][m] = mfma16x16x32<ADT>(av[k & 1][mt], bq[k & 1][m], part[mt][m]);
            }
          }
      }
      if constexpr (SB == 4) {
        if (q == 3) {
#pragma unroll
          for (int m = 0; m < NM; ++m) {
            uint32_t c;
            if constexpr (KF) c = (st.scw[m] >> (8 * h)) & 0xFFu;
            else c = st.scb[m][h];
            const float f = fp8x1(c);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][m] += part[mt][m] * f;
          }
        }
      }
    }
  };

  // pair tables of block b's expert: entry p = (level[p & (L-1)], level[p >> bits]) packed,
  // copied into every lane's bank slot (callers hold barriers on both sides)
  auto build_table = [&](int b) {
#pragma unroll
    for (int i = 0; i < NPAIR * 64 / (4 * kThreads); ++i) {
      const int base = i * 4 * kThreads + tid * 4;
      const int p = base >> 6, within = base & 63;
      const int t = GLU ? (within >> 5) : 0;
      const uint32_t v = (uint32_t)blk_lv[b][t][p & (L - 1)] | ((uint32_t)blk_lv[b][t][p >> BITS] << 16);
      *reinterpret_cast<u32x4*>(&tab[base]) = u32x4{v, v, v, v};
    }
  };

  // partial-sum exchange of items split between ranges (per wave, no workgroup barrier).
  // A range holds at most two split items, its first and its last: their partial tiles are
  // stored (device-coherent) when the item's part ends, and the arrival counts and sums wait
  // for the end of the range, where they hold up no streaming.
  const uint32_t npart_floats = G * 2 * kWaves * PF;
  auto part_off = [&](uint32_t gg, int which, int mt, int m) {   // byte offset of this lane's float4
    return (int)((((gg * 2 + which) * kWaves + wave) * PF + (mt * NM + m) * kWave * 4 + lane * 4) * 4);
  };
  auto real_rows = [&](int b, int mt) {    // does this lane hold any real slot row?
    const int r0 = b * BM + mt * 16 + 4 * lg;
    return min(min(slots[r0], slots[r0 + 1]), min(slots[r0 + 2], slots[r0 + 3])) < a.num_slots;
  };

  // stores of one finished item (reference order: acc * es; silu(g) * (u * es_u); * topk weight)
  auto store_item = [&](const Pos& p, int b) {
    const int nrow = p.pn * kRows + wave * 16 + ln;
    if (nrow >= a.N) return;
    const float es0 = blk_es[b][0], es1 = blk_es[b][NM - 1];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = b * BM + mt * 16 + 4 * lg + r;
        const int slot = slots[row];
        if (slot >= a.num_slots) continue;
        const int64_t at = (int64_t)slot * a.s_om + nrow;
        if constexpr (GLU) {
          const float gt = acc[mt][0][r] * es0;
          const float hv = gt / (1.0f + expf(-gt)) * (acc[mt][1][r] * es1);
          reinterpret_cast<uint16_t*>(a.out)[at] = (uint16_t)to_bits<ADT>(hv);
        } else {
          const float y = acc[mt][0][r] * es0 * slot_w[row];
          if (a.y16)
            reinterpret_cast<uint16_t*>(a.out)[at] = (uint16_t)to_bits<ADT>(y);
          else
            reinterpret_cast<float*>(a.out)[at] = y;
        }
      }
  };
  Pos split_p0{0, 0, 0}, split_p1{0, 0, 0};
  int split_b0 = 0, split_b1 = 0, n_split = 0;
  auto end_item = [&](const Pos& p, int b, bool full, bool first) {
    if (full) {
      store_item(p, b);
      return;
    }
    const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(a.part, npart_floats * 4);
    const int which = first ? 0 : 1;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (!real_rows(b, mt)) continue;
#pragma unroll
      for (int m = 0; m < NM; ++m)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mt][m]), rp, part_off(g, which, mt, m), 0,
                                               kCohere);
    }
    if (n_split == 0) {                // (named slots, not an indexed array: no scratch memory)
      split_p0 = p;
      split_b0 = b;
    } else {
      split_p1 = p;
      split_b1 = b;
    }
    ++n_split;
  };
  // One counter per split item, on its own 64-byte line (kWaves ints apart), bumped once per
  // workgroup after a barrier: every wave's partial tile is out before the count.
  auto finish_splits = [&]() {
    if (n_split == 0) return;            // (uniform: all waves share the range)
    __builtin_amdgcn_s_waitcnt(0);       // this wave's partial tiles are visible device-wide
    __syncthreads();                     // ... and every wave's
    uint32_t it[2];
    int g_lo[2], g_hi[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const Pos p = k == 0 ? split_p0 : split_p1;
      it[k] = (pm0 + p.pm) * nrt + p.pn;
      g_lo[k] = owner(it[k] * nun, U, G);
      g_hi[k] = owner(it[k] * nun + nun - 1, U, G);
    }
    if (tid == 0) {                      // both arrivals in flight together
      int old0 = 0, old1 = 0;
      old0 = __hip_atomic_fetch_add(a.counters + it[0] * kWaves, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (n_split > 1)
        old1 = __hip_atomic_fetch_add(a.counters + it[1] * kWaves, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool l0 = old0 == g_hi[0] - g_lo[0], l1 = n_split > 1 && old1 == g_hi[1] - g_lo[1];
      if (l0) __hip_atomic_store(a.counters + it[0] * kWaves, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (l1) __hip_atomic_store(a.counters + it[1] * kWaves, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      split_last[0] = l0;
      split_last[1] = l1;
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(a.part, npart_floats * 4);
    for (int k = 0; k < n_split; ++k) {
      if (!split_last[k]) continue;      // another workgroup finishes this item
      const Pos p = k == 0 ? split_p0 : split_p1;
      const int b = k == 0 ? split_b0 : split_b1;
      // sum the parts in range order
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (!real_rows(b, mt)) continue;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
          for (int gg = g_lo[k]; gg <= g_hi[k]; ++gg) {
            const int w = (U * gg / G) / nun == it[k] ? 0 : 1;
            const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, part_off(gg, w, mt, m), 0,
                                                                                             kCohere));
            t = gg == g_lo[k] ? v : t + v;
          }
          acc[mt][m] = t;
        }
      }
      store_item(p, b);
    }
  };

  // ---- prologue. Down requests the first trip's weights as soon as the blocks' experts are
  // staged, then the rest of the staging (expert scales, top-k weights, levels) and the first
  // trip's activation tiles (config 2, T=16: 26.0 -> 25.5 us); gate/up, whose first trip is
  // twice as large, requests the small loads first (the weights first measured 0.1-0.3 us
  // slower). The staged values are stored and the first block's pair tables built when they
  // arrive, then the first trip's tiles are published and the second trip's requested.
  Pos cp{0, (int)(item0 - pm0 * nrt), (int)(ub - item0 * nun)};
  Pos lp = cp;
  Stage<BITS, NM, SB, KF> st[P];
  int jl = 0;
  setup(lp);
  auto publish = [&](uint32_t* tiles) {        // this trip's activation tiles into the ring
#pragma unroll
    for (int d = 0; d < P; ++d)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) tiles[(d * 2 + h) * TILE + mt * 1024 + wave * 64 + lane] = ax[d][h][mt];
  };
  auto first_weights = [&]() {
#pragma unroll
    for (int d = 0; d < P; ++d) {
      if (d > 0 && lp.s == 0 && jl < n) setup(lp);
      load(lp.s, jl < n, st[d]);
      advance(lp);
      ++jl;
    }
  };
  constexpr int NLV = (MAXBLK * NM * L + kThreads - 1) / kThreads;   // staged values per thread
  constexpr int NSW = (MAXBLK * BM + kThreads - 1) / kThreads;
  static_assert(MAXBLK <= kThreads, "one thread per block's expert scales");
  if constexpr (!GLU) first_weights();
  __builtin_amdgcn_sched_barrier(0);
  const int e_own = tid < MAXBLK ? expert_of(tid) : -1;
  float es_v[NM], lv_v[NLV], sw_v[NSW];
#pragma unroll
  for (int m = 0; m < NM; ++m) es_v[m] = e_own >= 0 ? (m == 0 ? a.w0 : a.w1).expert_scale[e_own] : 0.f;
#pragma unroll
  for (int q = 0; q < NLV; ++q) {
    const int i = q * kThreads + tid;
    const int b = i / (NM * L), m = (i / L) % NM, c = i % L;
    const int e = i < MAXBLK * NM * L ? expert_of(b) : -1;
    lv_v[q] = e >= 0 ? (m == 0 ? a.w0 : a.w1).levels[(int64_t)e * L + c] : 0.f;
  }
#pragma unroll
  for (int q = 0; q < NSW; ++q) {
    const int r = q * kThreads + tid;
    sw_v[q] = (!GLU && r < MAXBLK * BM && slots[r] < a.num_slots) ? a.topk_w[slots[r]] : 0.f;
  }
  __builtin_amdgcn_sched_barrier(0);
  act_trip();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (GLU) first_weights();
  __builtin_amdgcn_sched_barrier(0);
  if (tid < MAXBLK) {
    blk_e[tid] = e_own;
#pragma unroll
    for (int m = 0; m < NM; ++m) blk_es[tid][m] = es_v[m];
  }
#pragma unroll
  for (int q = 0; q < NLV; ++q) {
    const int i = q * kThreads + tid;
    if (i < MAXBLK * NM * L) (&blk_lv[0][0][0])[i] = (uint16_t)to_bits<ADT>(lv_v[q]);
  }
  if constexpr (!GLU)
#pragma unroll
    for (int q = 0; q < NSW; ++q) {
      const int r = q * kThreads + tid;
      if (r < MAXBLK * BM) slot_w[r] = sw_v[q];
    }
  __syncthreads();                     // the staged plan is complete
  const int e_first = __builtin_amdgcn_readfirstlane(blk_e[0]);   // (a range starts at its block 0)
  if (e_first >= 0) build_table(0);
  __builtin_amdgcn_sched_barrier(0);
  publish(ring[0]);                    // (the plan's LDS under the ring is no longer read)
  __builtin_amdgcn_sched_barrier(0);
  act_trip();
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();                     // the first trip's tiles and the first tables are complete

  // ---- main loop: one trip of P units per iteration. Loads per trip, in order: per unit the
  // weights of the unit P ahead, then the activation tiles of the trip after next. The next
  // trip's tiles go into the other ring stage at the end, under one barrier per trip.
  int cur_b = 0, cur_e = e_first, e = e_first, sa = 0;     // block 0's tables are built
  bool first = true;
  for (int j0 = 0; j0 < n; j0 += P) {
    const int t = j0 / P;
    const uint32_t* tiles = ring[t & 1];
#pragma unroll
    for (int d = 0; d < P; ++d) {
      const int j = j0 + d;
      if (j < n) {
        const int b = min(cp.pm, MAXBLK - 1);
        if (b != cur_b) {                // a new block: its expert and pair tables
          cur_b = b;
          e = __builtin_amdgcn_readfirstlane(blk_e[b]);
          if (e >= 0 && e != cur_e) {
            if (cur_e >= 0) __syncthreads();   // the old tables' readers are done
            build_table(b);
            __syncthreads();
            cur_e = e;
          }
        }
        if (j == 0 || cp.s == 0) {
          sa = cp.s;
          first = j == 0;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int m = 0; m < NM; ++m) acc[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        if (e >= 0) {
          compute(cp.s, st[d], tiles + d * 2 * TILE);
          if (cp.s == nun - 1 || j == n - 1) end_item(cp, b, sa == 0 && cp.s == nun - 1, first);
        }
        advance(cp);
      }
      if (lp.s == 0 && jl < n) setup(lp);
      __builtin_amdgcn_sched_barrier(0);
      load(lp.s, jl < n, st[d]);
      __builtin_amdgcn_sched_barrier(0);
      advance(lp);
      ++jl;
    }
    publish(ring[(t + 1) & 1]);        // (its readers, two trips back, passed the last barrier)
    __builtin_amdgcn_sched_barrier(0);
    act_trip();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();                   // the next trip's tiles are complete
  }
  finish_splits();
}

}  // namespace bh
