// Fused HEX expert GEMMs on the CDNA4 matrix cores, and the k-slot reduction.
//
// Replaces the reference's _hex_moe_kernel (runtime/blackhole_runtime/hex_moe.py:109-151) in
// both roles (GLU gate/up with SiLU, and down with the top-k weight) and the torch sum at
// hex_moe.py:325. Designed for the decode regime, where a layer streams every routed expert's
// packed indices once and the matrix cores have room to spare:
//
//  * Work items are (expert block of the slot plan) x (row tile of 128 / k_split output rows).
//    The grid is persistent (two workgroups per compute unit); each workgroup takes a
//    contiguous range of the used items, so consecutive items mostly share an expert and its
//    LDS tables. Block experts and slot rows of the range are staged in LDS first.
//  * A workgroup has 8 waves (4 per SIMD at two workgroups per compute unit); they split the
//    tile's rows and, with k_split > 1, the inputs
//    (partials summed through LDS at the end of each item).
//  * Each lane streams the packed words of one whole 32-input block per row per step with one
//    128-bit load (4-bit; three dwords at 3-bit): row n = lane % 16, block 4 s + lane / 16, so a
//    step covers 128 inputs of 16 rows. Loads run D steps ahead of the math in registers, and
//    the pipeline runs across item boundaries, so HBM sees a steady stream of requests.
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

#include "hex_common.h"

namespace bh {

int check_proj(const bh_hex_proj* w, int64_t n_in, const char* who, int* block);

struct MoeArgs {
  const uint16_t* x;     // activations [rows, K] (bf16/f16 bits)
  int64_t s_xm;
  void* out;             // GLU: act [slots, N] (activation dtype); down: y [slots, N] float
  int64_t s_om;
  bh_hex_proj w0, w1;    // gate, up (GLU) or down (w0 only)
  const int32_t* sid;
  const int32_t* eid;
  const int32_t* npp;
  const int32_t* lookup;
  const float* topk_w;
  int64_t num_slots;
  int32_t n_experts;
  int32_t a_div;
  int32_t N, K;
  int32_t k_split;
  int32_t scale_words;   // block_scale rows allow 32-bit loads of 4 scales
};

// Four fp8 scales (one byte each) -> float, by the conversion instruction; a wave holding a
// 0x7F / 0xFF code (NaN for the instruction, +-480 for the reference formula) takes the formula.
__device__ __forceinline__ void fp8x4(uint32_t w, float f[4]) {
  const bool special = (((w & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u) != 0u;
  if (__builtin_expect(__ballot(special) != 0ull, 0)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = fp8_e4m3((w >> (8 * j)) & 0xFFu);
  } else {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    f[0] = lo[0]; f[1] = lo[1]; f[2] = hi[0]; f[3] = hi[1];
  }
}

__device__ __forceinline__ float fp8x1(uint32_t b) {
  const bool special = (b & 0x7Fu) == 0x7Fu;
  if (__builtin_expect(__ballot(special) != 0ull, 0)) return fp8_e4m3(b);
  return __builtin_amdgcn_cvt_f32_fp8((int)b, 0);
}

// Eight operands (two per dword, K order) for the codes of one 24/32-bit field.
template <int BITS>
__device__ __forceinline__ u32x4 lookup8(uint32_t f, uint32_t cb, const uint32_t* tab) {
  const char* base = reinterpret_cast<const char*>(tab);
  u32x4 b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t addr;
    if constexpr (BITS == 4) addr = __builtin_amdgcn_perm(f, cb, 0x0C0C0000u | ((4u + j) << 8));  // byte j << 8 | cb
    else addr = (((f >> (6 * j)) & 63u) << 8) | cb;
    b[j] = *reinterpret_cast<const uint32_t*>(base + addr);
  }
  return b;
}

template <int BITS, int MT, int NM>
struct Stage {
  uint32_t w[NM][4];     // 4-bit: the block's 4 words; 3-bit: its 3 words
  uint32_t sc[NM];       // block scales: 4 bytes (one per MFMA) or 1 byte (128-input block)
  u32x4 ax[MT][4];       // activation fragments of the 4 MFMAs
};

// Buffer resources and per-lane byte offsets of one work item (expert block x row tile). Each
// resource spans one expert's matrix (or the activations), so loads past its end return zero
// instead of faulting; rows past the matrix and padding slots read data whose results are
// never stored. The step offset goes in the scalar soffset, so a step costs no address math.
template <int MT, int NM>
struct ItemRes {
  __amdgpu_buffer_rsrc_t rw[NM];   // packed index words of the item's expert
  __amdgpu_buffer_rsrc_t rb[NM];   // its fp8 block scales
  int vw[NM], vb[NM];              // lane offsets: row n, block 4 s + lane / 16
  int vx[MT];                      // lane offsets into the activations: slot row, 8 inputs
};

constexpr int kRsrcWord3 = 0x00020000;   // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(bytes > 0x7FFFFFFF ? 0x7FFFFFFF : bytes), kRsrcWord3);
}

// Expert blocks a workgroup's item range may touch (their experts and slot rows are staged in
// LDS); the launch sizes the grid so no range needs more. At 16-slot blocks; 64 / MT in general.
constexpr int kMaxBlk16 = 64;

// Position in a workgroup's (item, step) sequence, advanced without divisions.
struct Pos {
  int pm;      // block, relative to the range's first block
  int pn;      // row tile
  int sidx;    // step of this wave within the item
};

// Prefetch depth D: steps of 128 inputs in flight per wave, also the chunk the main loop moves
// by. With 128 registers per lane (four waves per SIMD) the gate/up kernel keeps 2 steps in
// flight, the down kernel 3 (dividing the 6 steps of a 768-input row); 16 waves per compute
// unit keep about as many bytes in flight as 8 waves with twice the depth, and hide twice the
// latency of the decode-lookup-MFMA chain.
template <int MT, bool GLU>
constexpr int depth() { return GLU ? (MT == 1 ? 2 : 1) : (MT == 1 ? 3 : (MT == 2 ? 2 : 1)); }

// floats per lane that one pass of the k-split reduction moves through LDS
template <bool GLU>
__host__ __device__ constexpr int red_chunk() { return GLU ? 4 : 2; }

constexpr int kThreads = 512;      // 8 waves: 4 per SIMD with two workgroups per compute unit
constexpr int kWaves = kThreads / kWave;

constexpr int kOOR = 0x7FFF0000;   // byte offset past every resource: loads return zero, fetch nothing

template <int BITS, int ADT, bool GLU, int MT, int SB, bool KF>
__global__ __launch_bounds__(kThreads, (GLU && MT == 4) ? 2 : 4) void hex_moe_kernel(MoeArgs a) {
  constexpr int L = 1 << BITS;
  constexpr int NPAIR = 1 << (2 * BITS);
  constexpr int NM = GLU ? 2 : 1;
  constexpr int BM = 16 * MT;
  constexpr int NV = MT * NM * 4;                          // accumulator floats per lane
  constexpr int RCH = red_chunk<GLU>();                    // k-split partials per lane and pass
  constexpr int D = depth<MT, GLU>();
  constexpr int MAXBLK = kMaxBlk16 / MT;
  // Everything a work item needs besides its streamed weights and activations is staged in LDS
  // at the start, so the main loop issues no global load except the pipeline's, unconditionally
  // (the hardware's in-order load counter then waits exactly as long as the data needs).
  __shared__ __align__(16) uint32_t tab[NPAIR * 64];
  extern __shared__ __align__(16) float red[];    // k-split partials, sized at launch (block_m 16 only)
  __shared__ int slots[MAXBLK * BM];                               // slot rows of the range's blocks
  __shared__ float slot_w[GLU ? 1 : MAXBLK * BM];                  // their top-k weights (down)
  __shared__ int blk_e[MAXBLK];                                    // tier-local expert (-1: none)
  __shared__ float blk_es[MAXBLK][NM];                             // expert scales
  __shared__ uint16_t blk_lv[MAXBLK][NM][L];                       // levels in the activation dtype

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: steps and row tiles stay scalar
  const int KS = a.k_split, NWN = kWaves / KS;
  const int wn = wave % NWN, wk = wave / NWN, BN = 16 * NWN;
  const int nrt = (a.N + BN - 1) / BN;
  const int nb32 = a.K / kHexBlock;
  const int nsteps = (nb32 + 3) / 4;
  const int spw = (nsteps + KS - 1) / KS;                 // steps per wave per item (uniform)
  const int spw_p = (spw + D - 1) / D * D;                // padded to whole chunks
  const int s0 = wk * spw;

  // ---- this workgroup's contiguous range of items over the used blocks
  const int64_t used = (int64_t)a.npp[0] / BM;
  const int64_t items = used * nrt;
  const int64_t i0 = items * blockIdx.x / gridDim.x, i1 = items * (blockIdx.x + 1) / gridDim.x;
  const int nitems = (int)(i1 - i0);
  if (nitems <= 0) return;
  const int64_t pm0 = i0 / nrt;
  const int pn0 = (int)(i0 - pm0 * nrt);
  const int nblk = min((int)((i1 - 1) / nrt - pm0 + 1), MAXBLK);

  // ---- stage block metadata (entries past the range: no expert, padding slots)
  for (int b = tid; b < MAXBLK; b += kThreads) {
    int e = -1;
    if (b < nblk) {
      const int eg = a.eid[pm0 + b];
      e = (eg >= 0 && eg < a.n_experts) ? a.lookup[eg] : -1;
    }
    blk_e[b] = e;
#pragma unroll
    for (int m = 0; m < NM; ++m) blk_es[b][m] = e >= 0 ? (m == 0 ? a.w0 : a.w1).expert_scale[e] : 0.f;
  }
  for (int r = tid; r < MAXBLK * BM; r += kThreads) {
    const int slot = r < nblk * BM ? a.sid[pm0 * BM + r] : (int)a.num_slots;
    slots[r] = slot;
    if constexpr (!GLU) slot_w[r] = slot < a.num_slots ? a.topk_w[slot] : 0.f;
  }
  for (int i = tid; i < MAXBLK * NM * L; i += kThreads) {
    const int b = i / (NM * L), m = (i / L) % NM, c = i % L;
    int e = -1;
    if (b < nblk) {
      const int eg = a.eid[pm0 + b];
      e = (eg >= 0 && eg < a.n_experts) ? a.lookup[eg] : -1;
    }
    blk_lv[b][m][c] = e >= 0 ? (uint16_t)to_bits<ADT>((m == 0 ? a.w0 : a.w1).levels[(int64_t)e * L + c]) : 0;
  }
  __syncthreads();

  uint32_t cb[NM];
  if constexpr (GLU) {
    cb[0] = (lane & 31u) * 4u;
    cb[NM - 1] = 128u + (lane & 31u) * 4u;
  } else {
    cb[0] = lane * 4u;
  }
  auto advance = [&](Pos& p) {       // by one chunk
    p.sidx += D;
    if (p.sidx == spw_p) {
      p.sidx = 0;
      if (++p.pn == nrt) {
        p.pn = 0;
        ++p.pm;
      }
    }
  };

  // ---- load stream: buffer loads, per-item descriptors, the step in soffset
  ItemRes<MT, NM> R;
  const int x_rows = (int)((a.num_slots + a.a_div - 1) / a.a_div);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, (int64_t)x_rows * a.s_xm * 2);
  constexpr int WSTEP = 4 * BITS * 4;          // bytes of 4 blocks of one row
  auto setup = [&](const Pos& p) {
    const int b = min(p.pm, MAXBLK - 1);
    const int e = __builtin_amdgcn_readfirstlane(blk_e[b]);   // uniform: keeps descriptors scalar
    const int n = p.pn * BN + wn * 16 + ln;
    const bool rv = e >= 0 && n < a.N;               // rows past the matrix fetch nothing
    const int64_t ee = e >= 0 ? e : 0;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const bh_hex_proj& w = m == 0 ? a.w0 : a.w1;
      R.rw[m] = buffer_rsrc(w.idx + ee * w.s_ie, (int64_t)a.N * w.s_in * 4);
      R.rb[m] = buffer_rsrc(w.block_scale + ee * w.s_be, (int64_t)a.N * w.s_bn);
      R.vw[m] = rv ? (int)(n * w.s_in * 4) + lg * (BITS * 4) : kOOR;
      R.vb[m] = rv ? (int)(n * w.s_bn) : kOOR;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {                // padding slots fetch nothing
      const int slot = slots[b * BM + mt * 16 + ln];
      R.vx[mt] = (e >= 0 && slot < a.num_slots) ? (int)((int64_t)(slot / a.a_div) * a.s_xm * 2) + lg * 16 : kOOR;
    }
  };
  // step j (0..spw_p-1) of the load stream's item: padded steps read out of range
  auto load = [&](int j, Stage<BITS, MT, NM>& st) {
    const int sr = s0 + j;
    const bool real = j < spw && sr < nsteps;
    const int s = __builtin_amdgcn_readfirstlane(real ? sr : 0);
    const int ws = real ? s * WSTEP : kOOR, bs1 = real ? 4 * s : kOOR, bs4 = real ? s : kOOR;
    const int xs = real ? s * 256 : kOOR;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      if constexpr (BITS == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(R.rw[m], R.vw[m], ws, 0);
        st.w[m][0] = v[0]; st.w[m][1] = v[1]; st.w[m][2] = v[2]; st.w[m][3] = v[3];
      } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b96(R.rw[m], R.vw[m], ws, 0);
        st.w[m][0] = v[0]; st.w[m][1] = v[1]; st.w[m][2] = v[2]; st.w[m][3] = 0u;
      }
      if constexpr (SB == 1) {
        if (a.scale_words) {
          st.sc[m] = __builtin_amdgcn_raw_buffer_load_b32(R.rb[m], R.vb[m], bs1, 0);
        } else {
          uint32_t v = 0u;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(R.rb[m], R.vb[m] + q, bs1, 0) << (8 * q);
          st.sc[m] = v;
        }
      } else {
        st.sc[m] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(R.rb[m], R.vb[m], bs4, 0);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        st.ax[mt][q] = __builtin_amdgcn_raw_buffer_load_b128(rx, R.vx[mt] + q * 64, xs, 0);
  };

  // ---- compute stream
  f32x4 acc[MT][NM];
  auto compute = [&](int s, const Stage<BITS, MT, NM>& st) {
    uint32_t r[NM][4];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) r[m][j] = st.w[m][j];
      } else {   // the block's 96-bit stream as four 24-bit fields of 8 codes
        r[m][0] = st.w[m][0];
        r[m][1] = __builtin_amdgcn_alignbit(st.w[m][1], st.w[m][0], 24);
        r[m][2] = __builtin_amdgcn_alignbit(st.w[m][2], st.w[m][1], 16);
        r[m][3] = st.w[m][2] >> 8;
      }
      transpose_rows4(r[m]);     // r[m][q] = field lg of block 4 s + q
    }
    const int nq = KF ? 4 : min(4, nb32 - 4 * s);
    if constexpr (SB == 1) {
      float sf[NM][4];
#pragma unroll
      for (int m = 0; m < NM; ++m) fp8x4(st.sc[m], sf[m]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q < nq) {
          u32x4 b[NM];
#pragma unroll
          for (int m = 0; m < NM; ++m) b[m] = lookup8<BITS>(r[m][q], cb[m], tab);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int m = 0; m < NM; ++m) {
              const f32x4 p = mfma16x16x32<ADT>(st.ax[mt][q], b[m], f32x4{0.f, 0.f, 0.f, 0.f});
              acc[mt][m] += p * sf[m][q];
            }
        }
      }
    } else {
      f32x4 part[MT][NM];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int m = 0; m < NM; ++m) part[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q < nq) {
          u32x4 b[NM];
#pragma unroll
          for (int m = 0; m < NM; ++m) b[m] = lookup8<BITS>(r[m][q], cb[m], tab);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int m = 0; m < NM; ++m) part[mt][m] = mfma16x16x32<ADT>(st.ax[mt][q], b[m], part[mt][m]);
        }
      }
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const float sf = fp8x1(st.sc[m]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][m] += part[mt][m] * sf;
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

  // epilogue of one item (reference order: acc * es; silu(g) * (u * es_u); * topk weight)
  auto epilogue = [&](const Pos& p, int e) {
    if constexpr (MT == 1) {
      if (KS > 1) {
        // partials pass through LDS RCH floats per lane at a time, which keeps the area small
        // enough for two workgroups per compute unit beside the lookup tables
#pragma unroll
        for (int q = 0; q < NV / RCH; ++q) {
          __syncthreads();       // the previous pass's readers of red are done
          if (wk > 0) {
            float* dst = red + ((wk - 1) * NWN + wn) * RCH * 64;
#pragma unroll
            for (int i = 0; i < RCH; ++i) dst[i * 64 + lane] = acc[0][(q * RCH + i) / 4][(q * RCH + i) % 4];
          }
          __syncthreads();
          if (wk == 0) {
#pragma unroll
            for (int j = 1; j < 4; ++j) {    // k_split <= 4
              if (j < KS) {
                const float* src = red + ((j - 1) * NWN + wn) * RCH * 64;
#pragma unroll
                for (int i = 0; i < RCH; ++i) acc[0][(q * RCH + i) / 4][(q * RCH + i) % 4] += src[i * 64 + lane];
              }
            }
          }
        }
      }
    }
    if (wk != 0 || e < 0) return;
    const int n = p.pn * BN + wn * 16 + ln;
    if (n >= a.N) return;
    const int b = min(p.pm, MAXBLK - 1);
    const float es0 = blk_es[b][0], es1 = blk_es[b][NM - 1];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = b * BM + mt * 16 + 4 * lg + r;
        const int slot = slots[row];
        if (slot >= a.num_slots) continue;
        if constexpr (GLU) {
          const float g = acc[mt][0][r] * es0;
          const float h = g / (1.0f + expf(-g)) * (acc[mt][1][r] * es1);
          reinterpret_cast<uint16_t*>(a.out)[(int64_t)slot * a.s_om + n] = (uint16_t)to_bits<ADT>(h);
        } else {
          const float y = acc[mt][0][r] * es0 * slot_w[row];
          reinterpret_cast<float*>(a.out)[(int64_t)slot * a.s_om + n] = y;
        }
      }
  };

  // ---- one pipeline over (item, chunk of D steps): loads run one chunk ahead, across item
  // boundaries; chunks never straddle items, so control is per chunk, not per step
  const int cpi = spw_p / D;                               // chunks per item
  const int nchunks = nitems * cpi;
  Stage<BITS, MT, NM> st[D];
  Pos lp{0, pn0, 0}, cp{0, pn0, 0};
  setup(lp);
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, st[d]);
  advance(lp);
  int cur_b = -1;
  for (int c = 0; c < nchunks; ++c) {
    const int b = min(cp.pm, MAXBLK - 1);
    const int e = __builtin_amdgcn_readfirstlane(blk_e[b]);
    if (cp.sidx == 0) {
      if (e >= 0 && (cur_b < 0 || blk_e[cur_b] != e)) {
        __syncthreads();
        build_table(b);
        __syncthreads();
        cur_b = b;
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (lp.sidx == 0) setup(lp);
    const int sc = s0 + cp.sidx;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (e >= 0 && cp.sidx + d < spw && sc + d < nsteps) compute(sc + d, st[d]);
      load(lp.sidx + d, st[d]);
    }
    if (cp.sidx + D == spw_p) epilogue(cp, e);
    advance(cp);
    advance(lp);
  }
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

// Dynamic LDS for the k-split partials: one reduction pass of (k_split - 1) waves per row tile.
template <bool GLU, int MT>
static size_t red_bytes(int ks) {
  return ks > 1 ? (size_t)(ks - 1) * (kWaves / ks) * red_chunk<GLU>() * kWave * sizeof(float) : 16;
}

template <int BITS, int ADT, bool GLU, int MT>
static void launch_sb(int sb, dim3 grid, hipStream_t st, const MoeArgs& a) {
  const bool kf = (a.K / kHexBlock) % 4 == 0;     // whole 128-input steps: no tail checks
  const size_t shm = red_bytes<GLU, MT>(a.k_split);
  const dim3 block(kThreads);
  if (sb == 1) {
    if (kf) hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 1, true>), grid, block, shm, st, a);
    else hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 1, false>), grid, block, shm, st, a);
  } else {   // 128-input scale blocks imply whole steps
    hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 4, true>), grid, block, shm, st, a);
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

static bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Persistent grid: at most two workgroups per compute unit (64 KB pair tables each), never more
// than there are (expert block, row tile) items, and enough that no workgroup's contiguous item
// range spans more expert blocks than it stages in LDS (64 / MT).
static dim3 persistent_grid(int64_t num_blocks, int64_t n_out, int block_n, int mt) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  const int64_t items = num_blocks * cdiv(n_out, block_n);
  int64_t g = items < 2 * (int64_t)cus[dev] ? items : 2 * (int64_t)cus[dev];
  const int64_t min_g = cdiv(num_blocks, kMaxBlk16 / mt - 2);
  if (g < min_g) g = min_g;
  return dim3((unsigned)(g > 0 ? g : 1));
}

// Shared argument checks of the two fused entry points; fills the plan part of MoeArgs.
static int check_moe(const char* who, int32_t bits, int32_t adt, int64_t n_out, int64_t n_in, const int32_t* sid,
                     const int32_t* eid, int64_t num_blocks, const int32_t* npp, const int32_t* lookup,
                     int32_t n_experts, int64_t num_slots, const bh_hex_tile* tile, int* mt, int* sb, MoeArgs& a) {
  if (bits != 3 && bits != 4) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": bits must be 3 or 4");
  if (adt != BH_HEX_BF16 && adt != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": activations must be BF16 or F16");
  if (!tile) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null tile");
  if (tile->block_m != 16 && tile->block_m != 32 && tile->block_m != 64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m must be 16, 32 or 64");
  if (tile->k_split != 1 && tile->k_split != 2 && tile->k_split != 4)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": k_split must be 1, 2 or 4");
  if (tile->block_n != 128 / tile->k_split)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_n must be 128 / k_split");
  if (tile->k_split > 1 && tile->block_m != 16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": k_split > 1 needs block_m 16");
  if (n_out <= 0 || n_out > (1 << 30) || n_in > (1 << 30)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad width");
  if (n_experts <= 0 || num_slots < 0 || num_blocks < 0 || num_blocks > INT32_MAX)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad plan sizes");
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
  a.k_split = tile->k_split;
  (void)sb;
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
  const int64_t nb32 = n_in / kHexBlock;
  if (nb32 % 4 || w->s_bn % 4 || w->s_be % 4 || !aligned(w->block_scale, 4)) *words = 0;
  return BH_HEX_OK;
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_moe_glu(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                              const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out, int64_t n_in,
                              const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks,
                              const int32_t* npp, const int32_t* lookup, int32_t n_experts, int64_t num_slots,
                              int32_t a_div, const bh_hex_tile* tile, void* stream) {
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
  if (num_blocks == 0 || num_slots == 0) return BH_HEX_OK;
  a.x = reinterpret_cast<const uint16_t*>(x);
  a.s_xm = s_xm;
  a.out = act;
  a.s_om = s_am;
  a.w0 = *gate;
  a.w1 = *up;
  a.a_div = a_div;
  a.scale_words = words;
  const dim3 grid = persistent_grid(num_blocks, n_out, tile->block_n, mt);
  launch_moe<true>(bits, x_dtype, mt, sb, grid, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(who);
}

extern "C" int bh_hex_moe_down(const void* act, int32_t act_dtype, int64_t s_am, float* y, int64_t s_ym,
                               const bh_hex_proj* down, int32_t bits, int64_t n_out, int64_t n_in,
                               const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks,
                               const int32_t* npp, const int32_t* lookup, int32_t n_experts, int64_t num_slots,
                               const float* topk_w, const bh_hex_tile* tile, void* stream) {
  const char* who = "bh_hex_moe_down";
  MoeArgs a{};
  int mt = 0, sb = 0, words = 1;
  int rc = check_moe(who, bits, act_dtype, n_out, n_in, sorted_ids, expert_ids, num_blocks, npp, lookup, n_experts,
                     num_slots, tile, &mt, &sb, a);
  if (rc) return rc;
  if ((rc = proj_setup(who, down, bits, n_in, &sb, &words))) return rc;
  if (!act || !y || !topk_w) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  if (s_am % 8 || !aligned(act, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": act rows must be 16-byte aligned");
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
  const dim3 grid = persistent_grid(num_blocks, n_out, tile->block_n, mt);
  launch_moe<false>(bits, act_dtype, mt, sb, grid, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(who);
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
