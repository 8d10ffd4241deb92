// Fused HEX expert GEMMs on the CDNA4 matrix cores, and the k-slot reduction.
//
// Replaces the reference's _hex_moe_kernel (runtime/blackhole_runtime/hex_moe.py:109-151) in
// both roles (GLU gate/up with SiLU, and down with the top-k weight) and the torch sum at
// hex_moe.py:325. Designed for the decode regime, where a layer streams every routed expert's
// packed indices once and the matrix cores have room to spare:
//
//  * grid = (expert blocks of the slot plan) x (output row tiles). A workgroup of 4 waves owns
//    one expert block (16 * MT slots) and 64 / k_split output rows; the waves split the rows
//    and, with k_split > 1, the input dimension (partials summed through LDS at the end).
//  * Each lane streams the packed words of one whole 32-input block per row per step with one
//    128-bit load (4-bit; three dwords at 3-bit): row n = lane % 16, block 4 s + lane / 16, so a
//    step covers 128 inputs of 16 rows. A 4x4 transpose across the wave's rows (permlane swaps)
//    then gives each lane the 8 codes the 16x16x32 MFMA wants from it, with all 32 inputs of one
//    MFMA inside one HEX block, so every MFMA partial carries exactly one fp8 block scale.
//  * Codes resolve through a pair table in LDS: entry p = (level[p & (L-1)], level[p >> bits])
//    rounded to the activation dtype and packed, so one ds_read_b32 yields two operands. The
//    table has one copy per lane in its own bank (32 copies each for gate and up, 64 for down);
//    the read address is (pair << 8) | lane copy offset, one v_perm_b32 at 4 bits.
//  * fp32 partial of each block x its fp8 scale is added to the accumulator; the expert scale,
//    SiLU * up, and the top-k weight are applied in the epilogue, in the reference's order.
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

template <int BITS, int ADT, bool GLU, int MT, int SB>
__global__ __launch_bounds__(256, 2) void hex_moe_kernel(MoeArgs a) {
  constexpr int L = 1 << BITS;
  constexpr int NPAIR = 1 << (2 * BITS);
  constexpr int NM = GLU ? 2 : 1;
  constexpr int BM = 16 * MT;
  constexpr int NV = MT * NM * 4;                         // accumulator floats per lane
  constexpr int TAB = NPAIR * 64 > 192 * NV ? NPAIR * 64 : 192 * NV;
  __shared__ __align__(16) uint32_t tab[TAB];
  __shared__ uint32_t lvb[2][16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const int pid_m = blockIdx.x, pid_n = blockIdx.y;
  if ((int64_t)pid_m * BM >= (int64_t)a.npp[0]) return;
  const int eg = a.eid[pid_m];
  if (eg < 0 || eg >= a.n_experts) return;
  const int e = a.lookup[eg];
  if (e < 0) return;

  // ---- pair tables
  if (tid < NM * L) {
    const int t = tid / L, c = tid % L;
    const float* lv = t == 0 ? a.w0.levels : a.w1.levels;
    lvb[t][c] = to_bits<ADT>(lv[(int64_t)e * L + c]);
  }
  __syncthreads();
  for (int base = tid * 4; base < NPAIR * 64; base += 256 * 4) {
    const int p = base >> 6, within = base & 63;
    const int t = GLU ? (within >> 5) : 0;
    const uint32_t v = lvb[t][p & (L - 1)] | (lvb[t][p >> BITS] << 16);
    *reinterpret_cast<u32x4*>(&tab[base]) = u32x4{v, v, v, v};
  }
  __syncthreads();
  uint32_t cb[NM];
  if constexpr (GLU) {
    cb[0] = (lane & 31u) * 4u;
    cb[NM - 1] = 128u + (lane & 31u) * 4u;
  } else {
    cb[0] = lane * 4u;
  }

  // ---- work split
  const int KS = a.k_split, NWN = 4 / KS;
  const int wn = wave % NWN, wk = wave / NWN;
  const int n = pid_n * (16 * NWN) + wn * 16 + ln;
  const bool nvalid = n < a.N;
  const int nb32 = a.K / kHexBlock;
  const int nsteps = (nb32 + 3) / 4;
  const int chunk = (nsteps + KS - 1) / KS;
  const int s0 = wk * chunk, s1 = min(nsteps, s0 + chunk);

  const uint16_t* xrow[MT];
  bool avalid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int slot = a.sid[(int64_t)pid_m * BM + mt * 16 + ln];
    avalid[mt] = slot < a.num_slots;
    xrow[mt] = a.x + (int64_t)(avalid[mt] ? slot / a.a_div : 0) * a.s_xm;
  }
  const uint32_t* wp[NM];
  const uint8_t* bsp[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const bh_hex_proj& w = m == 0 ? a.w0 : a.w1;
    wp[m] = w.idx + (int64_t)e * w.s_ie + (int64_t)(nvalid ? n : 0) * w.s_in;
    bsp[m] = w.block_scale + (int64_t)e * w.s_be + (int64_t)(nvalid ? n : 0) * w.s_bn;
  }

  auto load = [&](int s, Stage<BITS, MT, NM>& st) {
    const int blk = 4 * s + lg;
    const bool bv = nvalid && blk < nb32;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      if constexpr (BITS == 4) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (bv) v = *reinterpret_cast<const u32x4*>(wp[m] + blk * 4);
        st.w[m][0] = v[0]; st.w[m][1] = v[1]; st.w[m][2] = v[2]; st.w[m][3] = v[3];
      } else {
#pragma unroll
        for (int j = 0; j < 3; ++j) st.w[m][j] = bv ? wp[m][blk * 3 + j] : 0u;
        st.w[m][3] = 0u;
      }
      if constexpr (SB == 1) {
        if (a.scale_words) {
          st.sc[m] = nvalid ? *reinterpret_cast<const uint32_t*>(bsp[m] + 4 * s) : 0u;
        } else {
          uint32_t v = 0u;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (nvalid && 4 * s + q < nb32) v |= (uint32_t)bsp[m][4 * s + q] << (8 * q);
          st.sc[m] = v;
        }
      } else {
        st.sc[m] = nvalid ? (uint32_t)bsp[m][s] : 0u;
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int bq = 4 * s + q;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (avalid[mt] && bq < nb32) v = *reinterpret_cast<const u32x4*>(xrow[mt] + bq * kHexBlock + lg * 8);
        st.ax[mt][q] = v;
      }
  };

  f32x4 acc[MT][NM];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[mt][m] = f32x4{0.f, 0.f, 0.f, 0.f};

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
    const int nq = min(4, nb32 - 4 * s);
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

  // ---- main loop, one step of prefetch
  Stage<BITS, MT, NM> st0, st1;
  if (s0 < s1) load(s0, st0);
  for (int s = s0; s < s1; s += 2) {
    if (s + 1 < s1) load(s + 1, st1);
    compute(s, st0);
    if (s + 1 < s1) {
      if (s + 2 < s1) load(s + 2, st0);
      compute(s + 1, st1);
    }
  }

  // ---- k-split partials through LDS
  __syncthreads();
  if (KS > 1) {
    float* red = reinterpret_cast<float*>(tab);
    if (wk > 0) {
      float* dst = red + (int64_t)((wk - 1) * NWN + wn) * NV * 64;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[((mt * NM + m) * 4 + r) * 64 + lane] = acc[mt][m][r];
    }
    __syncthreads();
    if (wk == 0) {
      for (int j = 1; j < KS; ++j) {
        const float* src = red + (int64_t)((j - 1) * NWN + wn) * NV * 64;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][m][r] += src[((mt * NM + m) * 4 + r) * 64 + lane];
      }
    }
  }
  if (wk != 0 || !nvalid) return;

  // ---- epilogue (reference order: acc * es; silu(g) * (u * es_u); * topk weight)
  const float es0 = a.w0.expert_scale[e];
  const float es1 = GLU ? a.w1.expert_scale[e] : 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int slot = a.sid[(int64_t)pid_m * BM + mt * 16 + 4 * lg + r];
      if (slot >= a.num_slots) continue;
      if constexpr (GLU) {
        const float g = acc[mt][0][r] * es0;
        const float h = g / (1.0f + expf(-g)) * (acc[mt][1][r] * es1);
        reinterpret_cast<uint16_t*>(a.out)[(int64_t)slot * a.s_om + n] = (uint16_t)to_bits<ADT>(h);
      } else {
        const float y = acc[mt][0][r] * es0 * a.topk_w[slot];
        reinterpret_cast<float*>(a.out)[(int64_t)slot * a.s_om + n] = y;
      }
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

template <int BITS, int ADT, bool GLU, int MT>
static void launch_sb(int sb, dim3 grid, hipStream_t st, const MoeArgs& a) {
  if (sb == 1) hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 1>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 4>), grid, dim3(256), 0, st, a);
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
  if (tile->block_n != 64 / tile->k_split)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_n must be 64 / k_split");
  if (n_out <= 0 || n_out > (1 << 30) || n_in > (1 << 30)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad width");
  if (n_experts <= 0 || num_slots < 0 || num_blocks < 0 || num_blocks > INT32_MAX)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad plan sizes");
  if (num_blocks > 0 && (!sid || !eid || !npp || !lookup))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null plan pointer");
  if (cdiv(n_out, tile->block_n) > 65535) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": too many row tiles");
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
  const dim3 grid((unsigned)num_blocks, (unsigned)cdiv(n_out, tile->block_n));
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
  const dim3 grid((unsigned)num_blocks, (unsigned)cdiv(n_out, tile->block_n));
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
