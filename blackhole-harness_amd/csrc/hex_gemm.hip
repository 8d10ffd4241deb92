// Fused HEX expert GEMMs for the prefill regime, on the CDNA4 matrix cores.
//
// Takes the place of the reference's _hex_moe_kernel (runtime/blackhole_runtime/hex_moe.py:109-151)
// in both roles (GLU gate/up with SiLU, down with the top-k weight) when every expert gets
// many slots. The reference sends such batches to its dequant path (hex_moe.py:357-371), which
// writes the whole bf16 weight set and reads it back; here the packed indices go straight from
// HBM to the matrix cores. The plan's expert blocks are 128 slots (block_m = 128).
//
//  * One workgroup per tile of 128 slots x R weight rows of one expert (R = 256 at 3 bits, 512 at
//    4 bits; the workgroup's waves per GemmShape below): down takes R output rows; GLU takes R / 2
//    outputs, i.e. the same rows of gate and of up. Each wave holds all 128 slots x 16 NG weight
//    rows (NG groups of 16; GLU: half gate, half the same up rows) in accumulator tiles, so every
//    weight is decoded by exactly one wave.
//  * The inputs run in steps of 128 (4 HEX blocks, 4 MFMA k-slices). A step's activation tile
//    (128 gathered slot rows x 128 inputs, 32 KB) is loaded once per workgroup and staged
//    through a two-stage LDS ring in the MFMA's fragment order, so every fragment read is one
//    conflict-free ds_read_b128.
//  * Each lane streams the packed words of one 32-input block per weight row group per step
//    (128-bit loads at 4 bits), one step ahead of the math. A 4x4 transpose across the wave's
//    rows gives each lane the 8 codes of its MFMA operand; the codes resolve through the
//    expert's pair table in LDS (two operands per ds_read_b32, one copy per lane slot).
//  * Order of operations, as in the decode kernels: operands are round(level); the fp32 partial
//    of each block times its fp8 scale is added to the accumulator; the expert scale, SiLU * up
//    and the top-k weight are applied in the epilogue in the reference's order.
//  * Workgroups are numbered so that each XCD (its own L2) takes a contiguous run of tiles:
//    the row tiles of a block (sharing its activation rows) and consecutive blocks of an expert
//    (sharing its weights) run on the same L2.
#include <string>
#include <type_traits>

#include "hex_fused.h"

namespace bh {

// The workgroup's shape, by bit width and scale block (SB 4: one fp8 scale per 128 inputs,
// SB 1: per 32). Four waves per SIMD where the registers allow: two weight-row groups of 16 per
// wave, at most 128 registers.
//  * 4 bits: 16 waves (one workgroup per compute unit: the 64 KB pair table) measured against 8
//    waves of two groups (two waves per SIMD): config 5 T=2048 1106 -> 943 us.
//  * 3 bits, SB 4: 8 waves, two workgroups per compute unit, against 4 waves of four groups (two
//    waves per SIMD, every activation fragment read feeding four groups, each m-tile's partials
//    scaled behind the next m-tile's MFMAs): config 3 427.8 -> 424.4 us over four runs. 16 waves
//    of two groups, one workgroup per compute unit, measured 424 -> 433 us.
//  * 3 bits, SB 1: 4 waves of four groups; the 8-wave shape spills there (config 3 with 32-input
//    scales 503 -> 532 us).
constexpr int kMaxNG = 4, kMaxChunks = 8;
template <int BITS, int SB>
struct GemmShape {
  static constexpr int WAVES = BITS == 4 ? 16 : (SB == 4 ? 8 : 4);   // waves of a workgroup
  static constexpr int NG = WAVES == 4 ? 4 : 2;    // weight-row groups of 16 per wave
  static constexpr int THREADS = WAVES * kWave;
  static constexpr int ROWS = WAVES * NG * 16;     // weight rows of a workgroup (256, or 512 at 4 bits)
  static constexpr int CHUNKS = 32 / WAVES;        // 1 KB chunks of a step's activation tile per wave
  static constexpr int MINW = NG == 2 ? 4 : 2;     // waves per SIMD
};
constexpr int kGM = 128;                // slots of a tile: one expert block of the plan
constexpr int kGK = 128;                // inputs per pipeline step
constexpr int kGTile = kGM * kGK / 2;   // dwords of one step's activation tile
constexpr int kXcds = 8;

// s_waitcnt operand that waits until at most n vector-memory loads are in flight (gfx9:
// vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima)
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int BITS, int SB, bool GLU>
constexpr int gemm_cols() { return GLU ? GemmShape<BITS, SB>::ROWS / 2 : GemmShape<BITS, SB>::ROWS; }   // outputs of a tile

template <int BITS, int ADT, bool GLU, int SB>
__global__ __launch_bounds__((GemmShape<BITS, SB>::THREADS), (GemmShape<BITS, SB>::MINW)) void hex_gemm_kernel(MoeArgs a,
                                                                                                   int n_tiles) {
  // (arrays below are sized by the non-dependent maxima kMaxNG / kMaxChunks: with sizes that
  // depend on BITS this compiler emits no host-side launch stub for the kernel)
  constexpr int kNG = GemmShape<BITS, SB>::NG;
  constexpr int kGWaves = GemmShape<BITS, SB>::WAVES;
  constexpr int kGThreads = GemmShape<BITS, SB>::THREADS;
  constexpr int kChunks = GemmShape<BITS, SB>::CHUNKS;
  constexpr int kCols = gemm_cols<BITS, SB, GLU>();
  constexpr int L = 1 << BITS;
  constexpr int NPAIR = 1 << (2 * BITS);
  constexpr int NM = GLU ? 2 : 1;
  constexpr int BLKB = BITS * 4;               // bytes of one 32-input block of one row
  using W = typename std::conditional<BITS == 4, u32x4, u32x3>::type;
  // Pair-table copies per entry: 64 at 4 bits; 32 at 3 bits, so that two workgroups fit in a
  // compute unit's LDS (a wave's table reads go to the banks in two halves of 32 lanes, so 32
  // copies keep down's reads conflict-free; GLU's gate and up tables get 16 copies each).
  constexpr int TC = BITS == 4 ? 64 : 32;
  constexpr int ES = TC == 64 ? 8 : 7;           // log2 of an entry's bytes
  static_assert((NPAIR * TC / 4) % kGThreads == 0, "the table build gives every thread whole 16-byte stores");
  static_assert(kGWaves * kChunks == 32 && 8 + kNG <= 16 && kChunks <= 8, "a step's loads fit its 16 m-tile slots");
  // Activation ring depth: tiles are loaded one step ahead of the math, as are the weight
  // words (two register sets). (Two steps ahead measured no faster.)
  constexpr int D = 2;
  // One LDS object with the pair table first: the table sits at LDS address 0, so table reads
  // need no base add (the 16-bit instruction offset cannot hold a base past 64 KB).
  struct Lds {
    uint32_t tab[NPAIR * TC];
    uint32_t atile[D][kGTile];   // the activation tile ring
    int slots[kGM];
    float slot_w[GLU ? 1 : kGM];
    uint16_t lvs[NM][L];
  };
  __shared__ __align__(16) Lds sm;
  uint32_t* const tab = sm.tab;
  int* const slots = sm.slots;
  float* const slot_w = sm.slot_w;
  auto& lvs = sm.lvs;

  // ---- the tile. Workgroup id runs on XCD id % 8 (round-robin dispatch). The tiles in use
  // (blocks within the padded length, known only here) are split evenly over the XCDs, each
  // XCD taking a contiguous run; XCD x holds at least as many workgroups as its share, and the
  // rest exit.
  const int used = (a.npp[0] / kGM) * n_tiles;
  const int xcd = blockIdx.x % kXcds, loc = blockIdx.x / kXcds;
  const int q8 = used / kXcds, r8 = used % kXcds;
  if (loc >= q8 + (xcd < r8 ? 1 : 0)) return;
  const int lin = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + loc;
  const int b = lin / n_tiles, nt = lin % n_tiles;
  const int eg = a.eid[b];
  if (eg < 0 || eg >= a.n_experts) return;
  const int e = a.lookup[eg];
  if (e < 0) return;

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nst = a.K / kGK;

  // ---- stage the block's slot rows, top-k weights and levels
  for (int r = tid; r < kGM; r += kGThreads) {
    const int s = a.sid[(int64_t)b * kGM + r];
    slots[r] = s;
    if constexpr (!GLU) slot_w[r] = s < a.num_slots ? a.topk_w[s] : 0.f;
  }
  for (int i = tid; i < NM * L; i += kGThreads) {
    const bh_hex_proj& w = i < L ? a.w0 : a.w1;
    lvs[i / L][i % L] = (uint16_t)to_bits<ADT>(w.levels[(int64_t)e * L + i % L]);
  }
  __syncthreads();

  // ---- load offsets. Activations: chunk c = i * waves + wave of a step's tile is m-tile c / 4,
  // k-slice c % 4; lane (ln, lg) reads inputs 32 (c % 4) + 8 lg .. + 7 of slot row
  // 16 (c / 4) + ln.
  const int x_rows = (int)((a.num_slots + a.a_div - 1) / a.a_div);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (int64_t)x_rows * a.s_xm * 2);
  uint32_t xo[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    const int c = i * kGWaves + wave;
    const int s = slots[(c >> 2) * 16 + ln];
    xo[i] = s < a.num_slots ? (uint32_t)((int64_t)(s / a.a_div) * a.s_xm * 2) + ((c & 3) * 32 + lg * 8) * 2 : kOOR;
  }
  // Weights: the wave's groups of 16 rows; lane (ln, lg) reads block lg of the step of row ln.
  // Down: rows R nt + 16 (NG wave + g). GLU: group g is gate (g < NG/2) or up, half h = g % (NG/2):
  // rows R/2 nt + 16 (NG/2 wave + h) of both, so a lane holds gate and up of the same outputs.
  constexpr int HG = kNG / 2;
  uint32_t vw[kMaxNG], vb[kMaxNG];
  uint32_t cb[kMaxNG];
  __amdgpu_buffer_rsrc_t rw[kMaxNG], rb[kMaxNG];
#pragma unroll
  for (int g = 0; g < kNG; ++g) {
    const int m = GLU ? g / HG : 0;
    const bh_hex_proj& w = m ? a.w1 : a.w0;
    rw[g] = buffer_rsrc(w.idx + (int64_t)e * w.s_ie, (int64_t)a.N * w.s_in * 4);
    rb[g] = buffer_rsrc(w.block_scale + (int64_t)e * w.s_be, (int64_t)a.N * w.s_bn);
    const int n = GLU ? nt * kCols + (wave * HG + g % HG) * 16 + ln : nt * kCols + (wave * kNG + g) * 16 + ln;
    vw[g] = n < a.N ? (uint32_t)((int64_t)n * w.s_in * 4) + lg * BLKB : kOOR;
    vb[g] = n < a.N ? (uint32_t)((int64_t)n * w.s_bn) : kOOR;
    cb[g] = GLU ? (uint32_t)m * (TC * 2) + (lane & (TC / 2 - 1)) * 4u : (lane & (TC - 1)) * 4u;
  }

  // a step's activation tile, straight into LDS (buffer loads with the LDS bit): chunk
  // i * waves + wave, 16 bytes per lane at lane * 16. Padding rows read out of range.
  auto load_a1 = [&](int st, int i, uint32_t* at) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)(at + (i * kGWaves + wave) * 256),
                                             16, voff(xo[i] + st * (kGK * 2)), 0, 0, 0);
  };
  auto load_a = [&](int st, uint32_t* at) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) load_a1(st, i, at);
  };
  auto load_w1 = [&](int st, int g, W& w, uint32_t& sc) {
    if constexpr (BITS == 4) ld_x4<0>(w, rw[g], vw[g] + st * 4 * BLKB);
    else ld_x3<0>(w, rw[g], vw[g] + st * 4 * BLKB);
    if constexpr (SB == 4) ld_u8<0>(sc, rb[g], vb[g] + st);
    else ld_x1<0>(sc, rb[g], vb[g] + 4 * st);
  };
  auto load_w = [&](int st, W (&ws)[kMaxNG], uint32_t (&sc)[kMaxNG]) {
#pragma unroll
    for (int g = 0; g < kNG; ++g) load_w1(st, g, ws[g], sc[g]);
  };

  W ws[2][kMaxNG];                   // weight words of this step and the next (ping-pong)
  uint32_t ss[2][kMaxNG];
  load_w(0, ws[0], ss[0]);
#pragma unroll
  for (int d = 0; d < D - 1; ++d) load_a(d < nst ? d : nst - 1, sm.atile[d]);

  // ---- the expert's pair table: entry p = (level[p & (L-1)], level[p >> bits]), TC copies
  // (GLU: the first half gate, the second up)
#pragma unroll
  for (int i = 0; i < NPAIR * TC / 4 / kGThreads; ++i) {
    const int base = (i * kGThreads + tid) * 4;
    const int p = base / TC, t = GLU ? (base % TC) / (TC / 2) : 0;
    const uint32_t v = (uint32_t)lvs[t][p & (L - 1)] | ((uint32_t)lvs[t][p >> BITS] << 16);
    *reinterpret_cast<u32x4*>(&tab[base]) = u32x4{v, v, v, v};
  }
  __builtin_amdgcn_s_waitcnt(vm_wait(kChunks * (D - 2)));   // step 0's loads have landed
  __syncthreads();

  f32x4 acc[8][kMaxNG];                     // [m-tile][group]
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int g = 0; g < kNG; ++g) acc[j][g] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One step (phase P = st % D): the loads of step st + D - 1 first (into the ring stage and
  // register set that step st - 1 used; past the end the last step repeats, so every load
  // stays unconditional), then the math of this one:
  // per half step (two k-slices) the groups' operands from the table, then per m-tile j the two
  // activation fragments (those of j + 1 are read before the MFMAs of j) and per group a
  // two-MFMA chain, whose block partial (128-input scales) is scaled into the accumulator; at
  // 32-input scales each MFMA's partial is scaled.
  auto step = [&](int st, auto phase) {
    constexpr int P = decltype(phase)::value;
    const uint32_t* at = sm.atile[st % D];
    const W (&cw)[kMaxNG] = ws[P];
    const uint32_t (&cs)[kMaxNG] = ss[P];
    const int sw = st + 1 < nst ? st + 1 : st;
    const int sa = st + D - 1 < nst ? st + D - 1 : nst - 1;
    uint32_t* const an = sm.atile[(st + D - 1) % D];
    // (scheduling barriers keep each phase's LDS reads ahead of the MFMAs that use them, and
    // the next step's loads spread over the m-tiles: issued back to back at the start of a
    // step, 64 loads per compute unit hold every wave at the memory pipe before its MFMAs)
    __builtin_amdgcn_sched_barrier(0);
    // the step's code fields and scales; the operands are looked up per half step (64 inputs,
    // k-slices 2 hq and 2 hq + 1), which keeps half the B operands live
    uint32_t r[kMaxNG][4];
    float f[kMaxNG][4];
#pragma unroll
    for (int g = 0; g < kNG; ++g) {
      fields<BITS>(cw[g], r[g]);         // r[g][q]: block 4 st + q
      fp8x4_nb(cs[g], f[g]);             // (at 128-input blocks the step's scale is byte 0; the
                                         // four-byte form also keeps the register allocation sane)
    }
    auto afrag = [&](int j, int hq, u32x4 (&av)[2]) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
        av[q] = *reinterpret_cast<const u32x4*>(at + ((j * 4 + 2 * hq + q) * 64 + lane) * 4);
    };
#pragma unroll
    for (int hq = 0; hq < 2; ++hq) {
      u32x4 bq[kMaxNG][2];
#pragma unroll
      for (int g = 0; g < kNG; ++g)
#pragma unroll
        for (int q = 0; q < 2; ++q) bq[g][q] = lookup8<BITS, ES>(r[g][2 * hq + q], cb[g], tab);
      u32x4 av[2][2];
      afrag(0, hq, av[0]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        if (j + 1 < 8) afrag(j + 1, hq, av[(j + 1) & 1]);
        // the next step's loads: tile chunks in the first half step (they must land in LDS by
        // the step's closing barrier, so they get the longer lead), words in the second (their
        // registers are waited for only where the next step reads them). Measured against the
        // opposite order: 3% (gate/up) and 4.5% (down) less time at a 4096-token prefill.
        const int t = hq * 8 + j;
        if (t < kChunks) load_a1(sa, t, an);
        else if (t >= 8 && t < 8 + kNG) load_w1(sw, t - 8, ws[1 - P][t - 8], ss[1 - P][t - 8]);
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 (&x)[2] = av[j & 1];
        if constexpr (SB == 4) {
          // the block's scale times the partial of each half step (one 128-input block per step)
          f32x4 p[kMaxNG];
#pragma unroll
          for (int g = 0; g < kNG; ++g) p[g] = mfma16x16x32<ADT>(x[0], bq[g][0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int g = 0; g < kNG; ++g) p[g] = mfma16x16x32<ADT>(x[1], bq[g][1], p[g]);
#pragma unroll
          for (int g = 0; g < kNG; ++g) acc[j][g] += p[g] * f[g][0];
        } else {
          // each k-slice partial times its block's scale
#pragma unroll
          for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int g = 0; g < kNG; ++g)
              acc[j][g] += mfma16x16x32<ADT>(x[q], bq[g][q], f32x4{0.f, 0.f, 0.f, 0.f}) * f[g][2 * hq + q];
        }
      }
    }

    // step st + 1's words and tile have landed (the tile loads issued after its words, for
    // D - 2 steps further on, stay in flight)
    __builtin_amdgcn_s_waitcnt(vm_wait(kChunks * (D - 2)));
    __syncthreads();                     // every wave's chunks of the next tile; this tile is free
  };
  // pairs of steps (the register set of a step is a compile-time constant), then the last one
  int st = 0;
  for (; st + 2 <= nst; st += 2) {
    step(st, std::integral_constant<int, 0>());
    step(st + 1, std::integral_constant<int, 1>());
  }
  if (st < nst) step(st, std::integral_constant<int, 0>());

  // ---- epilogue (reference order: acc * es; silu(g) * (u * es_u); * topk weight). The
  // outputs go through the (now free) activation ring, 64 KB, so that each slot row is written
  // with 16-byte stores, in passes of PR slot rows: GLU's tile in rows of kCols + 8 halves (the
  // padding staggers the banks); down's y in rows of kCols values whose 16-value column groups
  // are XORed with row bits 2-3 (the four row groups of a write land in distinct banks).
  const float es0 = a.w0.expert_scale[e], es1 = a.w1.expert_scale[e];
  uint32_t* const stage = sm.atile[0];                   // stages 0 and 1: 64 KB in a row
  auto at_rc = [](int row, int col) { return row * kCols + (col ^ (((row >> 2) & 3) << 4)); };
  if constexpr (GLU) {
    constexpr int RS = kCols + 8;                        // halves per staged row
    constexpr int PR = 32768 / RS >= kGM ? kGM : kGM / 2;
    constexpr int TPR = kCols / 8;                       // threads per row, 8 outputs (16 bytes) each
    static_assert(PR * RS <= 32768 && (PR * TPR) % kGThreads == 0 && kGM % PR == 0, "GLU staging passes");
    uint16_t* const st16 = reinterpret_cast<uint16_t*>(stage);
#pragma unroll
    for (int p = 0; p < kGM / PR; ++p) {
      if (p) __syncthreads();                            // the previous pass's readers are done
#pragma unroll
      for (int j = p * (PR / 16); j < (p + 1) * (PR / 16); ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int h = 0; h < HG; ++h) {
            const float gt = acc[j][h][r] * es0;
            const float hv = gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt)) * (acc[j][HG + h][r] * es1);
            st16[(j * 16 + 4 * lg + r - p * PR) * RS + (wave * HG + h) * 16 + ln] = (uint16_t)to_bits<ADT>(hv);
          }
        }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < PR * TPR / kGThreads; ++it) {
        const int row = it * (kGThreads / TPR) + tid / TPR, c = (tid % TPR) * 8;
        const int slot = slots[p * PR + row], col = nt * kCols + c;
        if (slot >= a.num_slots || col >= a.N) continue;
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)slot * a.s_om + col;
        const u32x4 v = *reinterpret_cast<const u32x4*>(st16 + row * RS + c);
        if (col + 8 <= a.N) {
          *reinterpret_cast<u32x4*>(dst) = v;
        } else {
          for (int q = 0; q < a.N - col; ++q) dst[q] = st16[row * RS + c + q];
        }
      }
    }
  } else if (a.y16) {
    // y in the activation dtype
    constexpr int PR = 32768 / kCols;                    // slot rows per pass
    constexpr int TPR = kCols / 8;
    static_assert((PR * TPR) % kGThreads == 0 && kGM % PR == 0 && PR % 16 == 0, "16-bit y staging passes");
    uint16_t* const st16 = reinterpret_cast<uint16_t*>(stage);
#pragma unroll
    for (int p = 0; p < kGM / PR; ++p) {
      if (p) __syncthreads();
#pragma unroll
      for (int j = p * (PR / 16); j < (p + 1) * (PR / 16); ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = j * 16 + 4 * lg + r - p * PR;  // within the pass
          const float w = slot_w[p * PR + row];
#pragma unroll
          for (int g = 0; g < kNG; ++g)
            st16[at_rc(row, (wave * kNG + g) * 16 + ln)] = (uint16_t)to_bits<ADT>(acc[j][g][r] * es0 * w);
        }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < PR * TPR / kGThreads; ++it) {
        const int row = it * (kGThreads / TPR) + tid / TPR, c = (tid % TPR) * 8;
        const int slot = slots[p * PR + row], col = nt * kCols + c;
        if (slot >= a.num_slots || col >= a.N) continue;
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)slot * a.s_om + col;
        const u32x4 v = *reinterpret_cast<const u32x4*>(st16 + at_rc(row, c));
        if (col + 8 <= a.N) {
          *reinterpret_cast<u32x4*>(dst) = v;
        } else {
          for (int q = 0; q < a.N - col; ++q) dst[q] = st16[at_rc(row, c) + q];
        }
      }
    }
  } else {
    // float32 y
    constexpr int PR = 16384 / kCols;                    // slot rows per pass
    constexpr int TPR = kCols / 4;                       // threads per row, 4 outputs (16 bytes) each
    static_assert((PR * TPR) % kGThreads == 0 && kGM % PR == 0 && PR % 16 == 0, "float32 y staging passes");
    float* const stf = reinterpret_cast<float*>(stage);
#pragma unroll
    for (int p = 0; p < kGM / PR; ++p) {
      if (p) __syncthreads();
#pragma unroll
      for (int j = p * (PR / 16); j < (p + 1) * (PR / 16); ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = j * 16 + 4 * lg + r - p * PR;
          const float w = slot_w[p * PR + row];
#pragma unroll
          for (int g = 0; g < kNG; ++g) stf[at_rc(row, (wave * kNG + g) * 16 + ln)] = acc[j][g][r] * es0 * w;
        }
      __syncthreads();
#pragma unroll
      for (int it = 0; it < PR * TPR / kGThreads; ++it) {
        const int row = it * (kGThreads / TPR) + tid / TPR, c = (tid % TPR) * 4;
        const int slot = slots[p * PR + row], col = nt * kCols + c;
        if (slot >= a.num_slots || col >= a.N) continue;
        float* dst = reinterpret_cast<float*>(a.out) + (int64_t)slot * a.s_om + col;
        const f32x4 v = *reinterpret_cast<const f32x4*>(stf + at_rc(row, c));
        if (col + 4 <= a.N) {
          *reinterpret_cast<f32x4*>(dst) = v;
        } else {
          for (int q = 0; q < a.N - col; ++q) dst[q] = stf[at_rc(row, c) + q];
        }
      }
    }
  }
}

// ----------------------------------------------------------------------------------- host side

template <int BITS, int ADT, bool GLU>
static void gemm_sb(int sb, dim3 grid, hipStream_t st, const MoeArgs& a, int n_tiles) {
  if (sb == 1)
    hipLaunchKernelGGL((hex_gemm_kernel<BITS, ADT, GLU, 1>), grid, dim3(GemmShape<BITS, 1>::THREADS), 0, st, a, n_tiles);
  else
    hipLaunchKernelGGL((hex_gemm_kernel<BITS, ADT, GLU, 4>), grid, dim3(GemmShape<BITS, 4>::THREADS), 0, st, a, n_tiles);
}

template <bool GLU>
static void gemm_launch(int bits, int adt, int sb, dim3 grid, hipStream_t st, const MoeArgs& a, int n_tiles) {
  if (bits == 4) {
    if (adt == BH_HEX_BF16) gemm_sb<4, BH_HEX_BF16, GLU>(sb, grid, st, a, n_tiles);
    else gemm_sb<4, BH_HEX_F16, GLU>(sb, grid, st, a, n_tiles);
  } else {
    if (adt == BH_HEX_BF16) gemm_sb<3, BH_HEX_BF16, GLU>(sb, grid, st, a, n_tiles);
    else gemm_sb<3, BH_HEX_F16, GLU>(sb, grid, st, a, n_tiles);
  }
}

// The 128-slot path: checks what it assumes beyond the shared checks, then launches one
// workgroup per (block, tile of outputs). Blocks past the plan's padded length, and blocks of
// experts outside the tier, exit at once.
int gemm_run(const char* who, bool glu, int bits, int adt, int sb, const MoeArgs& a, int64_t num_blocks,
             hipStream_t stream) {
  if (a.K % kGK) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m 128 needs n_in % 128 == 0");
  if (a.K > 16384) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m 128 takes n_in <= 16384");
  const bh_hex_proj* ws[2] = {&a.w0, &a.w1};
  for (int m = 0; m < (glu ? 2 : 1); ++m) {
    const bh_hex_proj& w = *ws[m];
    if ((int64_t)a.N * w.s_in * 4 > kMaxRecords || (int64_t)a.N * w.s_bn > kMaxRecords)
      return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": expert matrix over 2 GiB");
    if (sb == 1 && (w.s_bn % 4 || w.s_be % 4 || !aligned(w.block_scale, 4)))
      return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m 128 with 32-input scale blocks needs "
                                                             "4-byte aligned block_scale rows");
  }
  // output rows are written 16 bytes at a time
  if (a.s_om % ((glu || a.y16) ? 8 : 4) || !aligned(a.out, 16))
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m 128 needs 16-byte aligned output rows");
  const int64_t x_rows = cdiv(a.num_slots, a.a_div);
  if (x_rows * a.s_xm * 2 > kMaxRecords) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": activations over 2 GiB");
  // (a tile's outputs do not depend on the scale block: both 3-bit shapes cover 256 weight rows)
  static_assert(gemm_cols<3, 1, false>() == gemm_cols<3, 4, false>() && gemm_cols<4, 1, false>() == gemm_cols<4, 4, false>(),
                "tile widths per bit width");
  const int cols = bits == 4 ? (glu ? gemm_cols<4, 4, true>() : gemm_cols<4, 4, false>())
                             : (glu ? gemm_cols<3, 4, true>() : gemm_cols<3, 4, false>());
  const int64_t n_tiles = cdiv(a.N, cols);
  const int64_t wgs = num_blocks * n_tiles;
  if (wgs > INT32_MAX) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": plan too large");
  if (wgs == 0) return BH_HEX_OK;
  const dim3 grid((unsigned)wgs);
  if (glu) gemm_launch<true>(bits, adt, sb, grid, stream, a, (int)n_tiles);
  else gemm_launch<false>(bits, adt, sb, grid, stream, a, (int)n_tiles);
  return check_launch(who);
}

}  // namespace bh
