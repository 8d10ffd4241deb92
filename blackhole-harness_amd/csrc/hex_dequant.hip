// HEX dequant: one tier projection decoded into a stacked float/bf16/f16 output.
//
// Replaces the reference's _hex_dequant_kernel (runtime/blackhole_runtime/hex_moe.py:154-168)
// and the torch hex_dequant (blackhole/anatomy/hex.py:180-204). One thread decodes one
// 32-input bit stream of one row: it loads the stream's `bits` words (128-bit load at 4 bits),
// reads the 8/16 levels from LDS, and writes 32 outputs with 128-bit stores; consecutive threads
// take consecutive streams of a row, so loads and stores are coalesced. HBM-bound: per weight
// bits/8 + 1/B bytes in and 4 (f32) or 2 (bf16/f16) bytes out.
#include <string>

#include "hex_common.h"

namespace bh {

template <int BITS, int ODT, int ORDER>
__global__ __launch_bounds__(256) void hex_dequant_kernel(bh_hex_proj w, int64_t n_out, int64_t n_in, int32_t block,
                                                          const int32_t* __restrict__ expert_ids, void* __restrict__ out,
                                                          int64_t s_oe, int64_t s_on, int64_t row_off) {
  constexpr int L = 1 << BITS;
  __shared__ float lev[L];
  const int64_t e = blockIdx.y;
  if (threadIdx.x < L) lev[threadIdx.x] = w.levels[e * L + threadIdx.x];
  __syncthreads();
  const int64_t nb32 = n_in / kHexBlock;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_out * nb32) return;
  const int64_t o = t / nb32, b = t - o * nb32;

  uint32_t wd[BITS];
  const uint32_t* wp = w.idx + e * w.s_ie + o * w.s_in + b * BITS;
  if constexpr (BITS == 4) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(wp);
    wd[0] = v[0]; wd[1] = v[1]; wd[2] = v[2]; wd[3] = v[3];
  } else {
#pragma unroll
    for (int j = 0; j < BITS; ++j) wd[j] = wp[j];
  }
  const float f8 = fp8_e4m3(w.block_scale[e * w.s_be + o * w.s_bn + (b * kHexBlock) / block]);
  const float es = w.expert_scale[e];
  const float f8es = f8 * es;

  float vals[kHexBlock];
#pragma unroll
  for (int i = 0; i < kHexBlock; ++i) {
    const int off = i * BITS, wi = off / 32, sh = off % 32;
    uint32_t c = wd[wi] >> sh;
    if (sh + BITS > 32) c |= wd[wi + 1] << (32 - sh);
    const float v = lev[c & (L - 1)];
    float r;
    if constexpr (ORDER == BH_HEX_ORDER_R) r = v * f8es;
    else if constexpr (ORDER == BH_HEX_ORDER_D) r = (v * f8) * es;
    else r = bf16_to_f32(bf16_bits(v * f8));
    vals[i] = r;
  }

  const int64_t g = expert_ids ? (int64_t)expert_ids[e] : e;
  const int64_t ooff = g * s_oe + (row_off + o) * s_on + b * kHexBlock;
  if constexpr (ODT == BH_HEX_F32) {
    float* op = reinterpret_cast<float*>(out) + ooff;
#pragma unroll
    for (int i = 0; i < kHexBlock; i += 4) {
      f32x4 q = {vals[i], vals[i + 1], vals[i + 2], vals[i + 3]};
      *reinterpret_cast<f32x4*>(op + i) = q;
    }
  } else {
    uint16_t* op = reinterpret_cast<uint16_t*>(out) + ooff;
#pragma unroll
    for (int i = 0; i < kHexBlock; i += 8) {
      u32x4 q;
#pragma unroll
      for (int j = 0; j < 4; ++j) q[j] = to_bits<ODT>(vals[i + 2 * j]) | (to_bits<ODT>(vals[i + 2 * j + 1]) << 16);
      *reinterpret_cast<u32x4*>(op + i) = q;
    }
  }
}

template <int BITS, int ODT>
static int launch_dequant_order(int32_t order, dim3 grid, hipStream_t st, const bh_hex_proj& w, int64_t n_out,
                                int64_t n_in, int32_t block, const int32_t* ids, void* out, int64_t s_oe, int64_t s_on,
                                int64_t row_off) {
  switch (order) {
    case BH_HEX_ORDER_R:
      hipLaunchKernelGGL((hex_dequant_kernel<BITS, ODT, BH_HEX_ORDER_R>), grid, dim3(256), 0, st, w, n_out, n_in, block,
                         ids, out, s_oe, s_on, row_off);
      break;
    case BH_HEX_ORDER_D:
      hipLaunchKernelGGL((hex_dequant_kernel<BITS, ODT, BH_HEX_ORDER_D>), grid, dim3(256), 0, st, w, n_out, n_in, block,
                         ids, out, s_oe, s_on, row_off);
      break;
    default:
      hipLaunchKernelGGL((hex_dequant_kernel<BITS, ODT, BH_HEX_ORDER_T>), grid, dim3(256), 0, st, w, n_out, n_in, block,
                         ids, out, s_oe, s_on, row_off);
  }
  return check_launch("bh_hex_dequant");
}

template <int BITS>
static int launch_dequant_bits(int32_t out_dtype, int32_t order, dim3 grid, hipStream_t st, const bh_hex_proj& w,
                               int64_t n_out, int64_t n_in, int32_t block, const int32_t* ids, void* out, int64_t s_oe,
                               int64_t s_on, int64_t row_off) {
  switch (out_dtype) {
    case BH_HEX_F32:
      return launch_dequant_order<BITS, BH_HEX_F32>(order, grid, st, w, n_out, n_in, block, ids, out, s_oe, s_on,
                                                    row_off);
    case BH_HEX_BF16:
      return launch_dequant_order<BITS, BH_HEX_BF16>(order, grid, st, w, n_out, n_in, block, ids, out, s_oe, s_on,
                                                     row_off);
    default:
      return launch_dequant_order<BITS, BH_HEX_F16>(order, grid, st, w, n_out, n_in, block, ids, out, s_oe, s_on,
                                                    row_off);
  }
}

// Host-side checks of one projection shared by the entry points; *block receives the scale
// block size (inputs per fp8 scale).
int check_proj(const bh_hex_proj* w, int64_t n_in, const char* who, int* block) {
  if (!w || !w->idx || !w->block_scale || !w->expert_scale || !w->levels)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null HEX part pointer");
  if (n_in <= 0 || n_in % kHexBlock)
    return fail(BH_HEX_ERR_ASSERT, std::string(who) + ": input width " + std::to_string(n_in) + " is not a multiple of 32");
  if (w->block <= 0 || w->block % kHexBlock || n_in % w->block)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": scale block " + std::to_string(w->block) +
                                      " is not a multiple of 32 dividing the input width " + std::to_string(n_in));
  *block = w->block;
  return BH_HEX_OK;
}

}  // namespace bh

extern "C" int bh_hex_dequant(const bh_hex_proj* w, int32_t bits, int64_t n, int64_t n_out, int64_t n_in,
                              const int32_t* expert_ids, void* out, int32_t out_dtype, int64_t s_oe, int64_t s_on,
                              int64_t row_off, int32_t order, void* stream) {
  using namespace bh;
  if (bits != 3 && bits != 4) return fail(BH_HEX_ERR_UNSUPPORTED, "bh_hex_dequant: bits must be 3 or 4");
  if (out_dtype != BH_HEX_F32 && out_dtype != BH_HEX_BF16 && out_dtype != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, "bh_hex_dequant: out dtype must be F32, BF16 or F16");
  if (order < BH_HEX_ORDER_R || order > BH_HEX_ORDER_T) return fail(BH_HEX_ERR_VALUE, "bh_hex_dequant: bad order");
  if (n < 0 || n_out < 0) return fail(BH_HEX_ERR_VALUE, "bh_hex_dequant: negative size");
  if (!out) return fail(BH_HEX_ERR_VALUE, "bh_hex_dequant: null output");
  if (n == 0 || n_out == 0) return BH_HEX_OK;
  int block = 0;
  if (int rc = check_proj(w, n_in, "bh_hex_dequant", &block)) return rc;
  if ((w->s_ie % 4 || w->s_in % 4 || (reinterpret_cast<uintptr_t>(w->idx) & 15)) && bits == 4)
    return fail(BH_HEX_ERR_VALUE, "bh_hex_dequant: 4-bit idx rows must be 16-byte aligned");
  const int64_t per16 = out_dtype == BH_HEX_F32 ? 4 : 8;   // elements per 16 bytes
  if ((s_on % per16) || (s_oe % per16) || (reinterpret_cast<uintptr_t>(out) & 15))
    return fail(BH_HEX_ERR_VALUE, "bh_hex_dequant: output rows must be 16-byte aligned");
  const int64_t threads = n_out * (n_in / kHexBlock);
  const dim3 grid((unsigned)cdiv(threads, 256), (unsigned)n);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (bits == 4)
    return launch_dequant_bits<4>(out_dtype, order, grid, st, *w, n_out, n_in, block, expert_ids, out, s_oe, s_on,
                                  row_off);
  return launch_dequant_bits<3>(out_dtype, order, grid, st, *w, n_out, n_in, block, expert_ids, out, s_oe, s_on,
                                row_off);
}
