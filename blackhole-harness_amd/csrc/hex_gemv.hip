// The HEX MoE layer of one tier for a handful of slots (decode batches of a few tokens), as two
// matrix-vector launches: gate/up with SiLU, then down with the top-k weight and the k-slot sum
// folded in.
//
// Replaces, at these batches, the reference's align + two _hex_moe_kernel launches + sum
// (runtime/blackhole_runtime/hex_moe.py:304-325). With one or two tokens the layer is a few
// dependent memory round trips, and the expert-block kernels pay a slot plan, the partial-sum
// exchange of items split between workgroups, and a third launch for the sum. Here:
//
//  * gate/up: one wave per (slot, output row), grid (rows / 16, slots). Lane m takes 32-input
//    blocks m, m + 64, ... of the row (16 bytes of 4-bit codes, 12 of 3-bit, and the block's fp8
//    scale), so a row is one contiguous read across the wave. Codes resolve two at a time through
//    the expert's pair table in LDS (entry p = (level[p & (L-1)], level[p >> bits]) rounded to
//    the activation dtype, one dword), and one v_dot2 multiplies a pair with two activations in
//    float32. A block's partial times its fp8 scale adds to the lane's sum; the wave sum, the
//    expert scale and SiLU(gate) * up give act[slot, row], rounded to the activation dtype.
//  * down: a workgroup per (group of output rows, token), one wave per slot of the token. Lane
//    (g, b) takes 32-input block b of the slot's act row (held in registers for every row) and
//    of rows r = g, g + 64 / GS, ... of the group, GS lanes per row (GS = the act row's blocks,
//    rounded up to a power of two). The wave builds its slot's pair table in its own part of
//    LDS (from one level load, spread over the lanes by cross-lane reads: no barrier), then sums
//    each row as its weights arrive, times the block scales, the expert scale and the slot's
//    top-k weight. One barrier, then the k slots' partial sums of each row are added in slot
//    order and rounded once to the activation dtype: the top-k weight and the k-slot sum fold
//    into the launch (no per-slot y, no sum launch).
// The gate/up launch requests the first row's weights before it builds the pair tables and
// stages the activations in LDS, so the weights' HBM latency overlaps that set-up. Small loads
// are issued before large ones everywhere: a wait for a load also waits for every load issued
// before it. No slot plan: a slot's expert is its routing id. An expert that two slots share is
// read once per slot; the path is for batches where that costs less than the plan and the
// exchanges (the caller chooses).
#include <algorithm>
#include <string>

#include "hex_fused.h"

namespace bh {

constexpr int kGvGluWaves = 16;    // output rows of a gate/up workgroup (one per wave)
constexpr int kGvGluCs = 4;        // log2 of the copies of each gate/up pair-table entry (lane l
                                   // reads copy l % 16: four lanes share a copy)
constexpr int kGvDownLds = 65536;  // LDS of a down workgroup: its waves' tables and row sums
constexpr int kGvMaxK = 16;        // slots per token
constexpr int kGvMaxH = 4096;      // gate/up inputs (the staged activation row, 8 KB)
constexpr int kGvMaxI = 2048;      // down inputs (a row's blocks within one wave)

struct GemvArgs {
  const uint16_t* x;      // [T, H] activations (bf16 / f16 bits)
  int64_t s_xm;
  uint16_t* act;          // [T * k, I] gate/up output, activation dtype
  int64_t s_am;
  uint16_t* out;          // [T, H] layer output, activation dtype
  int64_t s_om;
  bh_hex_proj g, u, d;    // gate, up, down of the tier
  const void* ids;        // [T * k] routing ids (I32 / I64)
  int32_t ids_i64;
  const float* topk_w;    // [T * k]
  const int32_t* lookup;  // tier lookup [n_experts]
  int32_t n_experts;
  int32_t T, k, H, I;
  int32_t sb_shift;       // log2(inputs per fp8 scale / 32): 0 or 2
  int32_t down_cs;        // log2 of the copies of each down pair-table entry
};

constexpr int kGvDownMaxCs = 4;    // most copies of a down pair-table entry: 16

// The tier's expert of slot s, -1 for none (an id outside [0, n_experts) or another tier's).
__device__ __forceinline__ int slot_expert(const GemvArgs& a, int64_t s) {
  const int64_t id = a.ids_i64 ? reinterpret_cast<const int64_t*>(a.ids)[s] : reinterpret_cast<const int32_t*>(a.ids)[s];
  return (id >= 0 && id < a.n_experts) ? a.lookup[id] : -1;
}

// Two activations times two levels, in float32, added to c.
template <int ADT>
__device__ __forceinline__ float dot2(uint32_t lv, uint32_t xv, float c) {
  if constexpr (ADT == BH_HEX_BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, lv), __builtin_bit_cast(bf16x2, xv), c, false);
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, lv), __builtin_bit_cast(f16x2, xv), c, false);
  }
}

// Code pair p (inputs 2p, 2p + 1) of one 32-input block's little-endian bit stream.
template <int BITS>
__device__ __forceinline__ uint32_t pair_of(const uint32_t (&w)[4], int p) {
  if constexpr (BITS == 4) {
    return (w[p >> 2] >> ((p & 3) * 8)) & 0xFFu;
  } else {
    const int o = 6 * p, wi = o >> 5, sh = o & 31;
    const uint32_t v = sh + 6 <= 32 ? (w[wi] >> sh) : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
    return v & 63u;
  }
}

// One 32-input block: the sum over its 16 code pairs of pair-table entries times activation
// pairs (xa: the block's 32 activations, 8 per u32x4, low half first). Entry p, copy c of the
// table is dword (p << cs) + c.
template <int BITS, int ADT>
__device__ __forceinline__ float block_dot(const uint32_t (&w)[4], const u32x4 (&xa)[4], const uint32_t* tab, int cs,
                                           int copy) {
  float p0 = 0.f, p1 = 0.f;              // two chains: even and odd pairs
#pragma unroll
  for (int p = 0; p < 16; p += 2) {
    const uint32_t e0 = tab[(pair_of<BITS>(w, p) << cs) + copy];
    const uint32_t e1 = tab[(pair_of<BITS>(w, p + 1) << cs) + copy];
    p0 = dot2<ADT>(e0, xa[p >> 2][p & 3], p0);
    p1 = dot2<ADT>(e1, xa[(p + 1) >> 2][(p + 1) & 3], p1);
  }
  return p0 + p1;
}

// v from another lane of the same row of 16 (a DPP pattern, no LDS).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of G lanes (G = 8, 16, 32 or 64), the same value in every lane
// of the group: quad swaps, then half-row and row mirrors, then swaps of rows and of halves.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G == 8 || G == 16 || G == 32 || G == 64, "group of 8, 16, 32 or 64 lanes");
  v += dpp_f<0xB1>(v);                 // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);                 // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);                // row_half_mirror
  if constexpr (G >= 16) v += dpp_f<0x140>(v);   // row_mirror
  if constexpr (G >= 32) {
    uint32_t x = __builtin_bit_cast(uint32_t, v), y = x;
    swap16(x, y);                      // x: odd rows take the even rows' values; y: the reverse
    v = __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
  }
  if constexpr (G == 64) {
    uint32_t x = __builtin_bit_cast(uint32_t, v), y = x;
    swap32(x, y);
    v = __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
  }
  return v;
}

__device__ __forceinline__ float gv_wave_sum(float v) { return group_sum<kWave>(v); }

// Pair-table entry p of a level table.
template <int BITS, int ADT>
__device__ __forceinline__ uint32_t pair_entry(const float* levels, int p) {
  constexpr int L = 1 << BITS;
  return to_bits<ADT>(levels[p & (L - 1)]) | (to_bits<ADT>(levels[p >> BITS]) << 16);
}

// Activation rows in LDS are piece-major: the 16-byte piece q (inputs 8q .. 8q + 7) of block b of
// a row of nb blocks is u32x4 q * nb + b, so lanes reading consecutive blocks read consecutive
// 16 bytes (the block-major layout puts every fourth lane on the same banks).
__device__ __forceinline__ void lds_x4(u32x4 (&xa)[4], const u32x4* row, int b, int nb) {
#pragma unroll
  for (int q = 0; q < 4; ++q) xa[q] = row[q * nb + b];
}
__device__ __forceinline__ int piece_slot(int i, int nb) { return (i & 3) * nb + (i >> 2); }

// One gate/up row's weights for a lane: the codes and scale of its blocks b = lane + 64 m.
template <int IT>
struct GluRow {
  uint32_t wg[IT][4], wu[IT][4], sg[IT], su[IT];
};

// Requests row n's weights (nothing where the row or a block lies outside the matrix: the
// offsets are out of range, so every path issues the same loads).
template <int BITS, int IT>
__device__ __forceinline__ void glu_row_load(GluRow<IT>& r, const GemvArgs& a, __amdgpu_buffer_rsrc_t rg,
                                             __amdgpu_buffer_rsrc_t ru, __amdgpu_buffer_rsrc_t rbg,
                                             __amdgpu_buffer_rsrc_t rbu, int n, int lane, int nb) {
  const bool row = n < a.I;
#pragma unroll
  for (int m = 0; m < IT; ++m) {
    const int b = lane + kWave * m;
    const bool in = row && b < nb;
    const uint32_t og = in ? (uint32_t)(n * a.g.s_in + b * BITS) * 4u : kOOR;
    const uint32_t ou = in ? (uint32_t)(n * a.u.s_in + b * BITS) * 4u : kOOR;
    if constexpr (BITS == 4) {
      const u32x4 vg = __builtin_amdgcn_raw_buffer_load_b128(rg, voff(og), 0, 0);
      const u32x4 vu = __builtin_amdgcn_raw_buffer_load_b128(ru, voff(ou), 0, 0);
      r.wg[m][0] = vg[0]; r.wg[m][1] = vg[1]; r.wg[m][2] = vg[2]; r.wg[m][3] = vg[3];
      r.wu[m][0] = vu[0]; r.wu[m][1] = vu[1]; r.wu[m][2] = vu[2]; r.wu[m][3] = vu[3];
    } else {
      const u32x3 vg = __builtin_amdgcn_raw_buffer_load_b96(rg, voff(og), 0, 0);
      const u32x3 vu = __builtin_amdgcn_raw_buffer_load_b96(ru, voff(ou), 0, 0);
      r.wg[m][0] = vg[0]; r.wg[m][1] = vg[1]; r.wg[m][2] = vg[2]; r.wg[m][3] = 0u;
      r.wu[m][0] = vu[0]; r.wu[m][1] = vu[1]; r.wu[m][2] = vu[2]; r.wu[m][3] = 0u;
    }
    const int sbk = b >> a.sb_shift;
    uint32_t osg = in ? (uint32_t)(n * a.g.s_bn + sbk) : kOOR;
    uint32_t osu = in ? (uint32_t)(n * a.u.s_bn + sbk) : kOOR;
    asm volatile("" : "+v"(osg), "+v"(osu));   // (one load each, not one per side of the select)
    r.sg[m] = __builtin_amdgcn_raw_buffer_load_b8(rbg, voff(osg), 0, 0);
    r.su[m] = __builtin_amdgcn_raw_buffer_load_b8(rbu, voff(osu), 0, 0);
  }
}

// act[s, n] from row n's weights (the pair tables and the slot's activations in LDS).
template <int BITS, int ADT, int IT>
__device__ __forceinline__ void glu_row_dot(const GluRow<IT>& r, const GemvArgs& a, const uint32_t* tg,
                                            const uint32_t* tu, const u32x4* xs, int s, int n, int lane, int nb,
                                            float esg, float esu) {
  const int copy = lane & ((1 << kGvGluCs) - 1);
  float accg = 0.f, accu = 0.f;
#pragma unroll
  for (int m = 0; m < IT; ++m) {
    const int b = lane + kWave * m;
    if (b < nb) {
      u32x4 xa[4];
      lds_x4(xa, xs, b, nb);
      accg += block_dot<BITS, ADT>(r.wg[m], xa, tg, kGvGluCs, copy) * fp8x1_nb(r.sg[m]);
      accu += block_dot<BITS, ADT>(r.wu[m], xa, tu, kGvGluCs, copy) * fp8x1_nb(r.su[m]);
    }
  }
  accg = gv_wave_sum(accg);
  accu = gv_wave_sum(accu);
  if (lane == 0) {   // (reference order: acc * es; silu(g) * (u * es_u))
    const float gt = accg * esg;
    const float hv = gt / (1.0f + expf(-gt)) * (accu * esu);
    a.act[(int64_t)s * a.s_am + n] = (uint16_t)to_bits<ADT>(hv);
  }
}

// Grid (row groups, slots): workgroup g of slot s covers rows g * 16 + wave, then (LOOP) every
// gridDim.x * 16 rows after it, each wave requesting its next row before it computes the current.
// Without LOOP a wave computes one row and holds one row's weights (fewer registers, so more
// waves resident: for grids that fit the GPU in one round).
template <int BITS, int ADT, int IT, bool LOOP>
__global__ __launch_bounds__(kGvGluWaves * kWave) void gemv_glu_kernel(GemvArgs a) {
  constexpr int L = 1 << BITS, NP = L * L, C = 1 << kGvGluCs, NT = kGvGluWaves * kWave;
  static_assert(NP * C / 4 <= NT && kGvMaxH / 8 <= NT, "four copies of an entry and one activation piece per thread");
  __shared__ __align__(16) uint32_t tab[2][NP * C];
  __shared__ __align__(16) u32x4 xs[kGvMaxH / 8];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int s = blockIdx.y, t = s / a.k;
  const int e = __builtin_amdgcn_readfirstlane(slot_expert(a, s));
  if (e < 0) return;                    // (uniform: a slot of no expert of this tier writes nothing)
  const int stride = gridDim.x * kGvGluWaves;
  int n = blockIdx.x * kGvGluWaves + wave;
  const int nb = a.H / kHexBlock;
  // Loads in the order their values are needed (a wait for a load also waits for every load
  // issued before it): the level values of this thread's table entries, its piece of the
  // activation row, then the first row's weights.
  const int p = tid / (C / 4);           // this thread writes copies 4 (tid % (C / 4)) .. + 3 of entry p
  const bool has_entry = tid < NP * C / 4;
  float lv[4] = {0.f, 0.f, 0.f, 0.f};
  if (has_entry) {
    const float* lg = a.g.levels + (int64_t)e * L;
    const float* lu = a.u.levels + (int64_t)e * L;
    lv[0] = lg[p & (L - 1)];
    lv[1] = lg[p >> BITS];
    lv[2] = lu[p & (L - 1)];
    lv[3] = lu[p >> BITS];
  }
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x + (int64_t)t * a.s_xm, (int64_t)a.H * 2);
  const bool has_x = tid < a.H / 8;
  u32x4 xv = {0u, 0u, 0u, 0u};
  if (has_x) xv = __builtin_amdgcn_raw_buffer_load_b128(rx, voff((uint32_t)tid * 16u), 0, 0);
  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(a.g.idx + (int64_t)e * a.g.s_ie, (int64_t)a.I * a.g.s_in * 4);
  const __amdgpu_buffer_rsrc_t ru = buffer_rsrc(a.u.idx + (int64_t)e * a.u.s_ie, (int64_t)a.I * a.u.s_in * 4);
  const __amdgpu_buffer_rsrc_t rbg = buffer_rsrc(a.g.block_scale + (int64_t)e * a.g.s_be, (int64_t)a.I * a.g.s_bn);
  const __amdgpu_buffer_rsrc_t rbu = buffer_rsrc(a.u.block_scale + (int64_t)e * a.u.s_be, (int64_t)a.I * a.u.s_bn);
  // two row buffers: a wave requests row n + stride before it computes row n (the first row
  // alone before the barrier: more requests ahead of the table loads delay the tables)
  GluRow<IT> r0, r1;
  glu_row_load<BITS, IT>(r0, a, rg, ru, rbg, rbu, n, lane, nb);
  if (has_entry) {
    const uint32_t g = to_bits<ADT>(lv[0]) | (to_bits<ADT>(lv[1]) << 16);
    const uint32_t u = to_bits<ADT>(lv[2]) | (to_bits<ADT>(lv[3]) << 16);
    reinterpret_cast<u32x4*>(tab[0])[tid] = u32x4{g, g, g, g};
    reinterpret_cast<u32x4*>(tab[1])[tid] = u32x4{u, u, u, u};
  }
  if (has_x) xs[piece_slot(tid, nb)] = xv;
  __syncthreads();
  const float esg = a.g.expert_scale[e], esu = a.u.expert_scale[e];
  if constexpr (!LOOP) {
    if (n < a.I) glu_row_dot<BITS, ADT, IT>(r0, a, tab[0], tab[1], xs, s, n, lane, nb, esg, esu);
    return;
  }
  while (n < a.I) {                     // (wave-uniform; no barrier inside)
    glu_row_load<BITS, IT>(r1, a, rg, ru, rbg, rbu, n + stride, lane, nb);
    glu_row_dot<BITS, ADT, IT>(r0, a, tab[0], tab[1], xs, s, n, lane, nb, esg, esu);
    n += stride;
    if (n >= a.I) break;
    glu_row_load<BITS, IT>(r0, a, rg, ru, rbg, rbu, n + stride, lane, nb);
    glu_row_dot<BITS, ADT, IT>(r1, a, tab[0], tab[1], xs, s, n, lane, nb, esg, esu);
    n += stride;
  }
}

// Writes entries lane + 64 r of a pair table with 2^cs copies each; lvl holds level[lane]
// (lanes below 2^BITS).
template <int BITS, int ADT>
__device__ __forceinline__ void wave_pair_table(uint32_t* tab, float lvl, int lane, int cs) {
  constexpr int L = 1 << BITS, NP = L * L;
  const int lv_bits = __builtin_bit_cast(int, lvl);
#pragma unroll
  for (int r = 0; r < NP / kWave; ++r) {
    const int p = lane + kWave * r;
    const float lo = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((p & (L - 1)) * 4, lv_bits));
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((p >> BITS) * 4, lv_bits));
    const uint32_t v = to_bits<ADT>(lo) | (to_bits<ADT>(hi) << 16);
    if (cs == 1) {
      reinterpret_cast<u32x2*>(tab + (p << 1))[0] = u32x2{v, v};
    } else {
      for (int c = 0; c < (1 << cs); c += 4) reinterpret_cast<u32x4*>(tab + (p << cs) + c)[0] = u32x4{v, v, v, v};
    }
  }
}

// Grid (row groups of RW = NI * 64 / GS rows, tokens), k waves: wave j is slot t * k + j.
template <int BITS, int ADT, int GS, int NI>
__global__ __launch_bounds__(kGvMaxK * kWave) void gemv_down_kernel(GemvArgs a) {
  constexpr int L = 1 << BITS, NP = L * L, RPI = kWave / GS, RW = NI * RPI;
  static_assert(NP % kWave == 0 || NP == kWave, "pair-table entries spread evenly over a wave");
  extern __shared__ __align__(16) uint32_t dyn[];   // per wave its pair table [NP << cs]; then sums [k][RW]
  const int tid = threadIdx.x, lane = tid & 63;
  const int j = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = blockIdx.y, k = a.k, cs = a.down_cs;
  uint32_t* tab = dyn + ((j * NP) << cs);
  float* sums = reinterpret_cast<float*>(dyn + ((k * NP) << cs));
  const int g = lane / GS, b = lane % GS;
  const int nbk = a.I / kHexBlock;
  const bool has_b = b < nbk;
  const int h0 = blockIdx.x * RW;
  const int64_t s = (int64_t)t * k + j;
  // the slot's act block first (it needs no routing id), then the expert, its level, its rows
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.act + s * a.s_am, (int64_t)a.I * 2);
  u32x4 xa[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    xa[q] = __builtin_amdgcn_raw_buffer_load_b128(ra, voff(has_b ? (uint32_t)(b * 64 + q * 16) : kOOR), 0, 0);
  const int e = __builtin_amdgcn_readfirstlane(slot_expert(a, s));
  float part[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) part[i] = 0.f;
  float es = 0.f, tw = 0.f;
  if (e >= 0) {                         // (uniform over the wave)
    es = a.d.expert_scale[e];
    tw = a.topk_w[s];
    const float lvl = lane < L ? a.d.levels[(int64_t)e * L + lane] : 0.f;
    const __amdgpu_buffer_rsrc_t rd = buffer_rsrc(a.d.idx + (int64_t)e * a.d.s_ie, (int64_t)a.H * a.d.s_in * 4);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(a.d.block_scale + (int64_t)e * a.d.s_be, (int64_t)a.H * a.d.s_bn);
    uint32_t w[NI][4], sc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int h = h0 + RPI * i + g;
      const bool in = has_b && h < a.H;
      const uint32_t ow = in ? (uint32_t)(h * a.d.s_in + b * BITS) * 4u : kOOR;
      uint32_t os = in ? (uint32_t)(h * a.d.s_bn + (b >> a.sb_shift)) : kOOR;
      asm volatile("" : "+v"(os));
      if constexpr (BITS == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rd, voff(ow), 0, 0);
        w[i][0] = v[0]; w[i][1] = v[1]; w[i][2] = v[2]; w[i][3] = v[3];
      } else {
        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rd, voff(ow), 0, 0);
        w[i][0] = v[0]; w[i][1] = v[1]; w[i][2] = v[2]; w[i][3] = 0u;
      }
      sc[i] = __builtin_amdgcn_raw_buffer_load_b8(rb, voff(os), 0, 0);
    }
    wave_pair_table<BITS, ADT>(tab, lvl, lane, cs);
    const int copy = lane & ((1 << cs) - 1);
#pragma unroll
    for (int i = 0; i < NI; ++i) part[i] = block_dot<BITS, ADT>(w[i], xa, tab, cs, copy) * fp8x1_nb(sc[i]);
  }
  // each row's sum over its GS lanes, times the expert scale and the top-k weight (reference
  // order: acc * es, then * topk weight)
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    float v = part[i];
    v = group_sum<GS>(v);
    if (b == 0) sums[j * RW + RPI * i + g] = v * es * tw;
  }
  __syncthreads();
  if (tid < RW && h0 + tid < a.H) {
    float acc = 0.f;
    for (int q = 0; q < k; ++q) acc += sums[q * RW + tid];    // slot order
    a.out[(int64_t)t * a.s_om + h0 + tid] = (uint16_t)to_bits<ADT>(acc);
  }
}

// Dynamic LDS of the down kernel: k pair tables of 2^cs copies and the k slots' row sums.
static int64_t down_lds(int bits, int cs, int k, int rw) {
  return (int64_t)k * ((((int64_t)1 << (2 * bits)) << cs) * 4 + (int64_t)rw * 4);
}

// Lanes per row of the down kernel: the act row's blocks rounded up to a power of two (>= 8).
static int down_gs(int64_t inter) {
  const int64_t nbk = inter / kHexBlock;
  return nbk <= 8 ? 8 : nbk <= 16 ? 16 : nbk <= 32 ? 32 : 64;
}
static int down_iters(int) { return 4; }

// The most copies (up to 16) whose tables fit the down workgroup's LDS.
static int down_copies(int bits, int k, int64_t inter) {
  const int gs = down_gs(inter), rw = down_iters(gs) * kWave / gs;
  int cs = kGvDownMaxCs;
  while (cs > 1 && down_lds(bits, cs, k, rw) > kGvDownLds) --cs;
  return cs;
}

// Row groups of the gate/up grid: enough workgroups for every CU's resident workgroups over the
// slots, each wave's rows balanced (waves walk rows from the first they take, one row group apart).
static unsigned glu_groups(int resident, const GemvArgs& a) {
  const int64_t rows = cdiv(a.I, kGvGluWaves);
  const int64_t want = std::max<int64_t>(1, (int64_t)device_cus() * resident / ((int64_t)a.T * a.k));
  const int64_t per = cdiv(rows, std::min(rows, want));           // rows per wave
  return (unsigned)cdiv(rows, per);
}

// Workgroups of a kernel that one CU holds at once.
template <typename K>
static int resident_of(K kernel) {
  int r = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&r, kernel, kGvGluWaves * kWave, 0) != hipSuccess || r < 1) r = 1;
  return r;
}

// One row per wave when every row's wave fits the GPU at once; otherwise waves walk rows.
template <int BITS, int ADT, int IT>
static void glu_launch(hipStream_t st, const GemvArgs& a) {
  static const int res_one = resident_of(gemv_glu_kernel<BITS, ADT, IT, false>);
  static const int res_loop = resident_of(gemv_glu_kernel<BITS, ADT, IT, true>);
  const int64_t groups = cdiv(a.I, kGvGluWaves);
  if (groups * a.T * a.k <= (int64_t)device_cus() * res_one) {
    const dim3 grid((unsigned)groups, (unsigned)(a.T * a.k));
    hipLaunchKernelGGL((gemv_glu_kernel<BITS, ADT, IT, false>), grid, dim3(kGvGluWaves * kWave), 0, st, a);
  } else {
    const dim3 grid(glu_groups(res_loop, a), (unsigned)(a.T * a.k));
    hipLaunchKernelGGL((gemv_glu_kernel<BITS, ADT, IT, true>), grid, dim3(kGvGluWaves * kWave), 0, st, a);
  }
}

template <int BITS, int ADT, int GS>
static void down_launch(hipStream_t st, const GemvArgs& a) {
  constexpr int NI = 4, RW = NI * kWave / GS;
  const dim3 grid((unsigned)cdiv(a.H, RW), (unsigned)a.T), block((unsigned)(a.k * kWave));
  const unsigned lds = (unsigned)down_lds(BITS, a.down_cs, a.k, RW);
  hipLaunchKernelGGL((gemv_down_kernel<BITS, ADT, GS, NI>), grid, block, lds, st, a);
}

template <int BITS, int ADT>
static void gemv_launch(hipStream_t st, const GemvArgs& a) {
  if (a.H / kHexBlock <= kWave) glu_launch<BITS, ADT, 1>(st, a);
  else glu_launch<BITS, ADT, 2>(st, a);
  switch (down_gs(a.I)) {
    case 8: down_launch<BITS, ADT, 8>(st, a); break;
    case 16: down_launch<BITS, ADT, 16>(st, a); break;
    case 32: down_launch<BITS, ADT, 32>(st, a); break;
    default: down_launch<BITS, ADT, 64>(st, a); break;
  }
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_moe_gemv(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am, void* out,
                               int32_t out_dtype, int64_t s_om, const bh_hex_proj* gate, const bh_hex_proj* up,
                               const bh_hex_proj* down, int32_t bits, int64_t hidden, int64_t inter,
                               const void* topk_ids, int32_t ids_dtype, const float* topk_w, const int32_t* lookup,
                               int32_t n_experts, int64_t T, int32_t k, void* stream) {
  const char* who = "bh_hex_moe_gemv";
  if (bits != 3 && bits != 4) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": bits must be 3 or 4");
  if (x_dtype != BH_HEX_BF16 && x_dtype != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": activations must be BF16 or F16");
  if (out_dtype != x_dtype) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": out must have x's dtype");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ids dtype must be I32 or I64");
  if (T < 0 || k <= 0 || hidden <= 0 || inter <= 0 || n_experts <= 0)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes");
  if (k > kGvMaxK) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": at most 16 slots per token");
  if (hidden % kHexBlock || inter % kHexBlock)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": widths must be multiples of 32");
  if (hidden > kGvMaxH || inter > kGvMaxI)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": hidden at most 4096 and inter at most 2048");
  if (T * k > 65535) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": at most 65535 slots");
  if (T == 0) return BH_HEX_OK;
  if (!x || !act || !out || !gate || !up || !down || !topk_ids || !topk_w || !lookup)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  if (s_xm % 8 || s_am % 8 || !aligned(x, 16) || !aligned(act, 16))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": x and act rows must be 16-byte aligned");
  if (s_xm < hidden || s_am < inter || s_om < hidden)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": row strides below the widths");
  if ((T - 1) * s_xm * 2 + hidden * 2 > (int64_t)kMaxRecords)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": x over 2 GiB");
  int sb = 0, words = 1;
  if (int rc = proj_setup(who, gate, bits, inter, hidden, &sb, &words)) return rc;
  if (int rc = proj_setup(who, up, bits, inter, hidden, &sb, &words)) return rc;
  if (int rc = proj_setup(who, down, bits, hidden, inter, &sb, &words)) return rc;
  GemvArgs a{};
  a.x = reinterpret_cast<const uint16_t*>(x);
  a.s_xm = s_xm;
  a.act = reinterpret_cast<uint16_t*>(act);
  a.s_am = s_am;
  a.out = reinterpret_cast<uint16_t*>(out);
  a.s_om = s_om;
  a.g = *gate;
  a.u = *up;
  a.d = *down;
  a.ids = topk_ids;
  a.ids_i64 = ids_dtype == BH_HEX_I64;
  a.topk_w = topk_w;
  a.lookup = lookup;
  a.n_experts = n_experts;
  a.T = (int32_t)T;
  a.k = k;
  a.H = (int32_t)hidden;
  a.I = (int32_t)inter;
  a.down_cs = down_copies(bits, k, inter);
  a.sb_shift = sb == 4 ? 2 : 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (bits == 4) {
    if (x_dtype == BH_HEX_BF16) gemv_launch<4, BH_HEX_BF16>(st, a);
    else gemv_launch<4, BH_HEX_F16>(st, a);
  } else {
    if (x_dtype == BH_HEX_BF16) gemv_launch<3, BH_HEX_BF16>(st, a);
    else gemv_launch<3, BH_HEX_F16>(st, a);
  }
  return check_launch(who);
}
