// Fused HEX expert GEMMs on the CDNA4 matrix cores, and the k-slot reduction.
//
// Replaces the reference's _hex_moe_kernel (runtime/blackhole_runtime/hex_moe.py:109-151) in
// both roles (GLU gate/up with SiLU, and down with the top-k weight) and the torch sum at
// hex_moe.py:325. Designed for the decode regime, where a layer streams every routed expert's
// packed indices once and the matrix cores have room to spare:
//
//  * Units of work are (expert block of the slot plan, 256-row tile, 128-input step). The grid
//    is persistent, one 16-wave workgroup per compute unit, and workgroup g takes the contiguous
//    unit range [U g / G, U (g + 1) / G): every workgroup streams the same number of steps, and
//    consecutive units mostly share an expert and its LDS tables. An item (block, row tile)
//    split between workgroups is finished by the last of them to arrive, which adds the others'
//    partial sums (left in a workspace with device-coherent stores) in workgroup order, so the
//    result does not depend on timing.
//  * Each wave owns 16 rows of the tile. Each lane streams the packed words of one whole
//    32-input block per row per step with one 128-bit load (4-bit; three dwords at 3-bit):
//    row = lane % 16, block 4 s + lane / 16. Loads run P steps ahead of the math in registers,
//    across item boundaries, so HBM sees a steady stream of requests.
//  * The step's activation tile (16 slots x 128 inputs per 16-slot subtile) is fetched once per
//    workgroup, a dword per lane, and passed through a two-stage LDS ring to all 16 waves.
//  * A 4x4 transpose across the wave's rows (permlane swaps) gives each lane the 8 codes the
//    16x16x32 MFMA wants from it, with all 32 inputs of one MFMA inside one HEX block, so every
//    MFMA partial carries exactly one fp8 block scale.
//  * Codes resolve through a pair table in LDS: entry p = (level[p & (L-1)], level[p >> bits])
//    rounded to the activation dtype and packed, so one ds_read_b32 yields two operands. The
//    table has one copy per lane in its own bank (32 copies each for gate and up, 64 for down);
//    the read address is (pair << 8) | lane copy offset, one v_perm_b32 at 4 bits. It is
//    rebuilt only when the expert changes.
//  * The fp32 partial of each block times its fp8 scale is added to the accumulator; the expert
//    scale, SiLU * up, and the top-k weight are applied in the epilogue, in the reference's order.
// Weights therefore enter the matrix cores as round(level) and the block scale is applied to
// the float32 block partial, where the reference rounds level * fp8 to the activation dtype.
#include <string>
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

// Buffer descriptors of the weight stream's current item. Each spans one expert's matrix, so loads past its end return
// zero instead of faulting; rows past the matrix read out of range (nothing fetched) and are
// never stored. The unit offset goes in the scalar soffset.
template <int NM>
struct ItemRes {
  __amdgpu_buffer_rsrc_t rw[NM];   // packed index words of the item's expert
  __amdgpu_buffer_rsrc_t rb[NM];   // its fp8 block scales
  int vw[NM], vb[NM];              // lane offsets: row n, block lane / 16 of the unit
};

// The hot loop keeps every load unconditional and in a fixed order, so the compiler's waits
// for them stay partial (vmcnt(N), not 0).

// Expert blocks a workgroup's unit range may touch (their experts and slot rows are staged in
// LDS); the launch sizes the grid so no range needs more. At 16-slot blocks; 64 / MT in general.
constexpr int kMaxBlk16 = 64;
constexpr int kMaxExperts = 1024;        // global expert ids the tier lookup may take

constexpr int kThreads = 1024;           // 16 waves, one workgroup per compute unit
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 16 * kWaves;       // output rows of one work item: 16 per wave
constexpr int kMinUnits = 2;             // units per workgroup below which the grid shrinks

// Units per trip P: the weight loads of P units are in flight per wave ahead of the math, and
// the activation tiles of the next P units are fetched one trip ahead; one workgroup barrier
// per trip publishes them.
template <int MT, bool GLU>
constexpr int trip() { return GLU ? (MT == 1 ? 2 : 1) : (MT == 4 ? 1 : 2); }

// Position of a unit: block (relative to the range's first), row tile, unit within the item.
struct Pos {
  int pm, pn, s;
};

// Partial sums of one wave's 16 x BM tile, [mt][m][lane][4] floats.
template <int MT, int NM>
constexpr int part_floats() { return MT * NM * kWave * 4; }

// Work decomposition shared by the host (grid, workspace) and the kernel: units are
// (expert block, 256-row tile, 256-input unit) in that order; workgroup g takes units
// [U g / G, U (g + 1) / G). An item (block, row tile) split between workgroups is summed by the
// last of them to finish, in workgroup order, from partials in the workspace.
__device__ __forceinline__ int owner(int64_t u, int64_t U, int64_t G) {
  return (int)(((u + 1) * G + U - 1) / U - 1);
}

template <int BITS, int ADT, bool GLU, int MT, int SB, bool KF>
__global__ __launch_bounds__(kThreads) void hex_moe_kernel(MoeArgs a) {
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
  __shared__ __align__(16) uint32_t tab[NPAIR * 64];
  __shared__ __align__(16) uint32_t ring[2][P * 2 * TILE];
  __shared__ int lut[kMaxExperts];                                 // the tier lookup
  __shared__ int slots[MAXBLK * BM];                               // slot rows of the range's blocks
  __shared__ float slot_w[GLU ? 1 : MAXBLK * BM];                  // their top-k weights (down)
  __shared__ int blk_g[MAXBLK];                                    // global expert of each block
  __shared__ int blk_e[MAXBLK];                                    // its tier-local expert, -1 for none
  __shared__ float blk_es[MAXBLK][NM];                             // expert scales
  __shared__ uint16_t blk_lv[MAXBLK][NM][L];                       // levels in the activation dtype
  __shared__ int split_last[2];                                    // this workgroup finishes split item k

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: units and row tiles stay scalar
  const int nrt = (a.N + kRows - 1) / kRows;
  const int nb32 = a.K / kHexBlock;
  const int nun = (nb32 + 7) / 8;                              // units per item

  // ---- this workgroup's contiguous range of units over the used blocks
  const int64_t used = (int64_t)a.npp[0] / BM;
  const int64_t U = used * nrt * nun;
  // With between half and all as many items as workgroups, each workgroup takes one whole item:
  // no item is split, so no partial sums are exchanged. Otherwise the units are spread evenly
  // (no empty range), splitting items.
  const int64_t items = used * nrt;
  const bool whole = items <= (int64_t)gridDim.x && 2 * items >= (int64_t)gridDim.x;
  const int64_t G = whole ? items : min((int64_t)gridDim.x, U), g = blockIdx.x;
  if (g >= G) return;
  const int64_t ub = U * g / G, ue = U * (g + 1) / G;
  const int n = (int)(ue - ub);
  const int64_t item0 = ub / nun, item1 = (ue - 1) / nun;
  const int64_t pm0 = item0 / nrt;
  const int nblk = min((int)(item1 / nrt - pm0 + 1), MAXBLK);

  // ---- stage the plan: tier lookup, block experts, slot rows
  for (int i = tid; i < a.n_experts; i += kThreads) lut[i] = a.lookup[i];
  for (int b = tid; b < MAXBLK; b += kThreads) blk_g[b] = b < nblk ? a.eid[pm0 + b] : -1;
  for (int r = tid; r < MAXBLK * BM; r += kThreads)
    slots[r] = r < nblk * BM ? a.sid[pm0 * BM + r] : (int)a.num_slots;
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

  // ---- weight stream: buffer loads, per-item descriptors, the unit in soffset
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
      R.vw[m] = rv ? (int)(nrow * w.s_in * 4) + lg * BLKB : kOOR;
      R.vb[m] = rv ? (int)(nrow * w.s_bn) : kOOR;
    }
  };
  // loads of unit s of the current descriptors; dummy units (past the range) read out of range.
  // per matrix: the two steps' blocks, then the unit's scales
  // The whole byte offset goes in the range-checked VGPR offset (soffset 0): dummy units and
  // invalid rows sit past every resource.
  auto load = [&](int s_, bool real, Stage<BITS, NM, SB, KF>& st) {
    const int s = __builtin_amdgcn_readfirstlane(real ? s_ : 0);
    const int ws = real ? s * USTEP : kOOR;
    const int bs = real ? (SB == 1 ? 8 : 2) * s : kOOR;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int vw = R.vw[m] + ws, vb = R.vb[m] + bs;
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
  const int x_rows = (int)((a.num_slots + a.a_div - 1) / a.a_div);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (int64_t)x_rows * a.s_xm * 2);
  // lane dword of a step's tile: wave w, lane l -> slot l / 4 of the subtile, inputs
  // 32 (w / 4) + 8 (w % 4) + 2 (l % 4) of the step (the fragment layout the MFMA reads)
  const int xcol = (wave >> 2) * 64 + (wave & 3) * 16 + (lane & 3) * 4;
  int vx[MT];
  int ax_b = -1;
  auto act_rows = [&](int b) {
    const int e = expert_of(b);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {            // padding slots fetch nothing
      const int slot = slots[b * BM + mt * 16 + (lane >> 2)];
      vx[mt] = (e >= 0 && slot < a.num_slots) ? (int)((int64_t)(slot / a.a_div) * a.s_xm * 2) + xcol : kOOR;
    }
  };
  uint32_t ax[P][2][MT];
  Pos ap{0, (int)(item0 - pm0 * nrt), (int)(ub - item0 * nun)};
  int ja = 0;
  auto act_trip = [&]() {                        // loads of the next P units' tiles
    int xs[P][2], vxd[P][MT];
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
      for (int h = 0; h < 2; ++h) xs[d][h] = __builtin_amdgcn_readfirstlane(real ? (2 * ap.s + h) * 256 : kOOR);
      advance(ap);
      ++ja;
    }
#pragma unroll
    for (int d = 0; d < P; ++d)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) ld_x1<0>(ax[d][h][mt], rx, vxd[d][mt] + xs[d][h]);
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

  // partial-sum exchange of items split between workgroups (per wave, no workgroup barrier).
  // A workgroup holds at most two split items, the first and the last of its range: their
  // partial tiles are stored (device-coherent) when the item's part ends, and the arrival
  // counts and sums wait for the end of the range, where they hold up no streaming.
  const int64_t npart_floats = G * 2 * kWaves * PF;
  auto part_off = [&](int64_t gg, int which, int mt, int m) {   // byte offset of this lane's float4
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
        if constexpr (GLU) {
          const float gt = acc[mt][0][r] * es0;
          const float hv = gt / (1.0f + expf(-gt)) * (acc[mt][1][r] * es1);
          reinterpret_cast<uint16_t*>(a.out)[(int64_t)slot * a.s_om + nrow] = (uint16_t)to_bits<ADT>(hv);
        } else {
          const float y = acc[mt][0][r] * es0 * slot_w[row];
          reinterpret_cast<float*>(a.out)[(int64_t)slot * a.s_om + nrow] = y;
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
    int64_t it[2];
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
      // sum the parts in workgroup order
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

  // ---- prologue: the rest of the staging (its waits leave nothing in flight), then the
  // pipeline's first loads in the loop's order: activation tiles, weights, and the first trip's
  // tiles published
  for (int b = tid; b < MAXBLK; b += kThreads) {
    const int e = expert_of(b);
    blk_e[b] = e;
#pragma unroll
    for (int m = 0; m < NM; ++m) blk_es[b][m] = e >= 0 ? (m == 0 ? a.w0 : a.w1).expert_scale[e] : 0.f;
  }
  if constexpr (!GLU)
    for (int r = tid; r < MAXBLK * BM; r += kThreads) slot_w[r] = slots[r] < a.num_slots ? a.topk_w[slots[r]] : 0.f;
  for (int i = tid; i < MAXBLK * NM * L; i += kThreads) {
    const int b = i / (NM * L), m = (i / L) % NM, c = i % L;
    const int e = expert_of(b);
    blk_lv[b][m][c] = e >= 0 ? (uint16_t)to_bits<ADT>((m == 0 ? a.w0 : a.w1).levels[(int64_t)e * L + c]) : 0;
  }
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
  __builtin_amdgcn_sched_barrier(0);
  act_trip();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < P; ++d) {
    if (d > 0 && lp.s == 0 && jl < n) setup(lp);
    load(lp.s, jl < n, st[d]);
    advance(lp);
    ++jl;
  }
  __builtin_amdgcn_sched_barrier(0);
  publish(ring[0]);
  __builtin_amdgcn_sched_barrier(0);
  act_trip();
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();                     // the first trip's tiles and the staged plan are complete

  // ---- main loop: one trip of P units per iteration. Loads per trip, in order: per unit the
  // weights of the unit P ahead, then the activation tiles of the trip after next. The next
  // trip's tiles go into the other ring stage at the end, under one barrier per trip.
  int cur_e = -1, cur_b = -1, e = -1, sa = 0;
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
  __builtin_amdgcn_s_waitcnt(0);       // no load of this wave is left in flight at exit
}

// ----------------------------------------------------------------------------------- reduction

template <int ODT, int IDT>
__global__ __launch_bounds__(256) void moe_reduce_kernel(const float* __restrict__ y, int64_t s_ym,
                                                         const void* __restrict__ ids, int32_t n_experts, int32_t k,
                                                         int64_t H, void* __restrict__ out, int64_t s_ot) {
  const int64_t t = blockIdx.y;
  const int64_t h = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (h >= H) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < k; ++j) {
    const int64_t s = t * k + j;
    int64_t id;
    if constexpr (IDT == BH_HEX_I64) id = reinterpret_cast<const int64_t*>(ids)[s];
    else id = reinterpret_cast<const int32_t*>(ids)[s];
    if (id < 0 || id >= n_experts) continue;
    acc += *reinterpret_cast<const f32x4*>(y + s * s_ym + h);
  }
  if constexpr (ODT == BH_HEX_F32) {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + t * s_ot + h) = acc;
  } else {
    u32x2 v;
    v[0] = to_bits<ODT>(acc[0]) | (to_bits<ODT>(acc[1]) << 16);
    v[1] = to_bits<ODT>(acc[2]) | (to_bits<ODT>(acc[3]) << 16);
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(out) + t * s_ot + h) = v;
  }
}

// ----------------------------------------------------------------------------------- host side

template <int BITS, int ADT, bool GLU, int MT>
static void launch_sb(int sb, dim3 grid, hipStream_t st, const MoeArgs& a) {
  // whole 256-input units with aligned scale rows: no tail checks, one load per unit's scales
  const bool kf = (a.K / kHexBlock) % 8 == 0 && a.scale_words;
  const dim3 block(kThreads);
  if (sb == 1) {
    if (kf) hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 1, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 1, false>), grid, block, 0, st, a);
  } else {
    if (kf) hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 4, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 4, false>), grid, block, 0, st, a);
  }
}

template <int BITS, int ADT, bool GLU>
static void launch_mt(int mt, int sb, dim3 grid, hipStream_t st, const MoeArgs& a) {
  if (mt == 1) launch_sb<BITS, ADT, GLU, 1>(sb, grid, st, a);
  else if (mt == 2) launch_sb<BITS, ADT, GLU, 2>(sb, grid, st, a);
  else launch_sb<BITS, ADT, GLU, 4>(sb, grid, st, a);
}

template <bool GLU>
static void launch_moe(int bits, int adt, int mt, int sb, dim3 grid, hipStream_t st, const MoeArgs& a) {
  if (bits == 4) {
    if (adt == BH_HEX_BF16) launch_mt<4, BH_HEX_BF16, GLU>(mt, sb, grid, st, a);
    else launch_mt<4, BH_HEX_F16, GLU>(mt, sb, grid, st, a);
  } else {
    if (adt == BH_HEX_BF16) launch_mt<3, BH_HEX_BF16, GLU>(mt, sb, grid, st, a);
    else launch_mt<3, BH_HEX_F16, GLU>(mt, sb, grid, st, a);
  }
}

int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Persistent grid: one workgroup per compute unit, fewer when the plan's units (an upper bound
// from num_blocks) would give a workgroup fewer than kMinUnits units, and enough that no
// workgroup's range spans more expert blocks than it stages in LDS (64 / MT).
static int64_t moe_grid(int64_t num_blocks, int64_t n_out, int64_t n_in, int mt) {
  const int64_t units = num_blocks * cdiv(n_out, kRows) * cdiv(cdiv(n_in, kHexBlock), 8);
  int64_t g = cdiv(units, kMinUnits);
  if (g > device_cus()) g = device_cus();
  const int64_t min_g = cdiv(num_blocks, kMaxBlk16 / mt - 2);
  if (g < min_g) g = min_g;
  return g > 0 ? g : 1;
}

// Workspace of one launch: arrival counters (one per item, 64 bytes apart) and partial-sum tiles
// (two per workgroup and wave), as two separate buffers so calls of any shape can share them.
struct Workspace {
  int64_t counters, partials;      // int32 counters, float partials
};

static Workspace workspace_layout(int64_t num_blocks, int64_t n_out, int64_t n_in, int mt, bool glu) {
  Workspace w;
  w.counters = num_blocks * cdiv(n_out, kRows) * kWaves;
  w.partials = moe_grid(num_blocks, n_out, n_in, mt) * 2 * kWaves * (int64_t)mt * (glu ? 2 : 1) * kWave * 4;
  return w;
}

// Shared argument checks of the two fused entry points; fills the plan part of MoeArgs.
static int check_moe(const char* who, int32_t bits, int32_t adt, int64_t n_out, int64_t n_in, const int32_t* sid,
                     const int32_t* eid, int64_t num_blocks, const int32_t* npp, const int32_t* lookup,
                     int32_t n_experts, int64_t num_slots, const bh_hex_tile* tile, int* mt, int* sb, MoeArgs& a) {
  if (bits != 3 && bits != 4) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": bits must be 3 or 4");
  if (adt != BH_HEX_BF16 && adt != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": activations must be BF16 or F16");
  if (!tile) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null tile");
  if (tile->block_m != 16 && tile->block_m != 32 && tile->block_m != 64 && tile->block_m != 128)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m must be 16, 32, 64 or 128");
  if (tile->block_n != kRows || tile->k_split != 1)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_n must be 256 and k_split 1");
  if (n_out <= 0 || n_out > (1 << 30) || n_in > (1 << 30)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad width");
  if (n_experts <= 0 || num_slots < 0 || num_blocks < 0 || num_blocks > INT32_MAX)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad plan sizes");
  if (n_experts > kMaxExperts)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": at most 1024 experts");
  if (num_blocks > 0 && (!sid || !eid || !npp || !lookup))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null plan pointer");
  *mt = tile->block_m / 16;
  a.sid = sid;
  a.eid = eid;
  a.npp = npp;
  a.lookup = lookup;
  a.n_experts = n_experts;
  a.num_slots = num_slots;
  a.N = (int32_t)n_out;
  a.K = (int32_t)n_in;
  (void)sb;
  return BH_HEX_OK;
}

// Points the kernel at the caller's workspace.
static int attach_workspace(const char* who, int32_t* counters, int64_t n_counters, float* partials,
                            int64_t n_partials, int64_t num_blocks, int64_t n_out, int64_t n_in, int mt, bool glu,
                            MoeArgs& a, dim3* grid) {
  const Workspace w = workspace_layout(num_blocks, n_out, n_in, mt, glu);
  if (!counters || !partials || n_counters < w.counters || n_partials < w.partials)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": workspace smaller than bh_hex_moe_workspace() asks");
  if (!aligned(partials, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": partials must be 16-byte aligned");
  if (w.partials * 4 > 0x7FFFFFFF) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": plan too large");
  a.counters = counters;
  a.part = partials;
  *grid = dim3((unsigned)moe_grid(num_blocks, n_out, n_in, mt));
  return BH_HEX_OK;
}

static int proj_setup(const char* who, const bh_hex_proj* w, int bits, int64_t n_in, int* sb, int* words) {
  int block = 0;
  if (int rc = check_proj(w, n_in, who, &block)) return rc;
  if (block != 32 && block != 128)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": fused kernels take scale blocks of 32 or 128 inputs");
  if (*sb && *sb != block / 32) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": gate and up scale blocks differ");
  *sb = block / 32;
  if (bits == 4 && (w->s_ie % 4 || w->s_in % 4 || !aligned(w->idx, 16)))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": 4-bit idx rows must be 16-byte aligned");
  // a unit's scales in one load: 8 bytes at 32-input blocks, 2 bytes at 128-input blocks
  const int sw = block == 32 ? 8 : 2;
  if (w->s_bn % sw || w->s_be % sw || !aligned(w->block_scale, sw)) *words = 0;
  return BH_HEX_OK;
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_moe_glu(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                              const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out, int64_t n_in,
                              const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks,
                              const int32_t* npp, const int32_t* lookup, int32_t n_experts, int64_t num_slots,
                              int32_t a_div, const bh_hex_tile* tile, int32_t* counters, int64_t n_counters,
                              float* partials, int64_t n_partials, void* stream) {
  const char* who = "bh_hex_moe_glu";
  MoeArgs a{};
  int mt = 0, sb = 0, words = 1;
  int rc = check_moe(who, bits, x_dtype, n_out, n_in, sorted_ids, expert_ids, num_blocks, npp, lookup, n_experts,
                     num_slots, tile, &mt, &sb, a);
  if (rc) return rc;
  if ((rc = proj_setup(who, gate, bits, n_in, &sb, &words))) return rc;
  if ((rc = proj_setup(who, up, bits, n_in, &sb, &words))) return rc;
  if (a_div <= 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": a_div must be positive");
  if (!x || !act) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null activation pointer");
  if (s_xm % 8 || !aligned(x, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": x rows must be 16-byte aligned");
  if (cdiv(num_slots, a_div) * s_xm * 2 > 0x7FFFFFFF) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": x over 2 GiB");
  if (num_blocks == 0 || num_slots == 0) return BH_HEX_OK;
  a.x = reinterpret_cast<const uint16_t*>(x);
  a.s_xm = s_xm;
  a.out = act;
  a.s_om = s_am;
  a.w0 = *gate;
  a.w1 = *up;
  a.a_div = a_div;
  a.scale_words = words;
  if (mt == kGemmMt) return gemm_run(who, true, bits, x_dtype, sb, a, num_blocks, reinterpret_cast<hipStream_t>(stream));
  dim3 grid;
  if ((rc = attach_workspace(who, counters, n_counters, partials, n_partials, num_blocks, n_out, n_in, mt, true, a,
                             &grid))) return rc;
  launch_moe<true>(bits, x_dtype, mt, sb, grid, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(who);
}

extern "C" int bh_hex_moe_down(const void* act, int32_t act_dtype, int64_t s_am, float* y, int64_t s_ym,
                               const bh_hex_proj* down, int32_t bits, int64_t n_out, int64_t n_in,
                               const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks,
                               const int32_t* npp, const int32_t* lookup, int32_t n_experts, int64_t num_slots,
                               const float* topk_w, const bh_hex_tile* tile, int32_t* counters, int64_t n_counters,
                               float* partials, int64_t n_partials, void* stream) {
  const char* who = "bh_hex_moe_down";
  MoeArgs a{};
  int mt = 0, sb = 0, words = 1;
  int rc = check_moe(who, bits, act_dtype, n_out, n_in, sorted_ids, expert_ids, num_blocks, npp, lookup, n_experts,
                     num_slots, tile, &mt, &sb, a);
  if (rc) return rc;
  if ((rc = proj_setup(who, down, bits, n_in, &sb, &words))) return rc;
  if (!act || !y || !topk_w) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  if (s_am % 8 || !aligned(act, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": act rows must be 16-byte aligned");
  if (num_slots * s_am * 2 > 0x7FFFFFFF) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": act over 2 GiB");
  if (num_blocks == 0 || num_slots == 0) return BH_HEX_OK;
  a.x = reinterpret_cast<const uint16_t*>(act);
  a.s_xm = s_am;
  a.out = y;
  a.s_om = s_ym;
  a.w0 = *down;
  a.w1 = *down;
  a.topk_w = topk_w;
  a.a_div = 1;
  a.scale_words = words;
  if (mt == kGemmMt) return gemm_run(who, false, bits, act_dtype, sb, a, num_blocks, reinterpret_cast<hipStream_t>(stream));
  dim3 grid;
  if ((rc = attach_workspace(who, counters, n_counters, partials, n_partials, num_blocks, n_out, n_in, mt, false, a,
                             &grid))) return rc;
  launch_moe<false>(bits, act_dtype, mt, sb, grid, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(who);
}

extern "C" int bh_hex_moe_workspace(int64_t num_blocks, int64_t n_out, int64_t n_in, int32_t block_m, int32_t glu,
                                    int64_t* n_counters, int64_t* n_partials) {
  if (num_blocks < 0 || n_out <= 0 || n_in <= 0 || !n_counters || !n_partials)
    return fail(BH_HEX_ERR_VALUE, "bh_hex_moe_workspace: bad arguments");
  if (block_m != 16 && block_m != 32 && block_m != 64 && block_m != 128)
    return fail(BH_HEX_ERR_UNSUPPORTED, "bh_hex_moe_workspace: block_m must be 16, 32, 64 or 128");
  if (block_m / 16 == kGemmMt) {     // the 128-slot kernels need no workspace
    *n_counters = 0;
    *n_partials = 0;
    return BH_HEX_OK;
  }
  const Workspace w = workspace_layout(num_blocks, n_out, n_in, block_m / 16, glu != 0);
  *n_counters = w.counters;
  *n_partials = w.partials;
  return BH_HEX_OK;
}

extern "C" int bh_hex_moe_reduce(const float* y, int64_t s_ym, const void* topk_ids, int32_t ids_dtype,
                                 int32_t n_experts, int64_t T, int32_t k, int64_t H, void* out, int32_t out_dtype,
                                 int64_t s_ot, void* stream) {
  const char* who = "bh_hex_moe_reduce";
  if (T < 0 || k <= 0 || H <= 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes");
  if (H % 4 || s_ym % 4 || s_ot % 4 || !aligned(y, 16) || !aligned(out, 16))
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": rows must be 16-byte aligned with H % 4 == 0");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ids dtype must be I32 or I64");
  if (T == 0) return BH_HEX_OK;
  if (T > 65535) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": more than 65535 tokens");
  const dim3 grid((unsigned)cdiv(H, 1024), (unsigned)T);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define BH_RED(ODT, IDT) \
  hipLaunchKernelGGL((moe_reduce_kernel<ODT, IDT>), grid, dim3(256), 0, st, y, s_ym, topk_ids, n_experts, k, H, out, s_ot)
  if (out_dtype == BH_HEX_F32) {
    if (ids_dtype == BH_HEX_I64) BH_RED(BH_HEX_F32, BH_HEX_I64); else BH_RED(BH_HEX_F32, BH_HEX_I32);
  } else if (out_dtype == BH_HEX_BF16) {
    if (ids_dtype == BH_HEX_I64) BH_RED(BH_HEX_BF16, BH_HEX_I64); else BH_RED(BH_HEX_BF16, BH_HEX_I32);
  } else if (out_dtype == BH_HEX_F16) {
    if (ids_dtype == BH_HEX_I64) BH_RED(BH_HEX_F16, BH_HEX_I64); else BH_RED(BH_HEX_F16, BH_HEX_I32);
  } else {
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": out dtype must be F32, BF16 or F16");
  }
#undef BH_RED
  return check_launch(who);
}
