// Device helpers shared by the HEX kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "bh_hex.h"

namespace bh {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x3 __attribute__((ext_vector_type(3)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr int kHexBlock = 32;     // inputs per bit stream

// ----------------------------------------------------------------------------------- scalars

// fp8 e4m3 code -> float by the kernels' formula: exponent 0 gives mt * 2^-9, otherwise
// (1 + mt / 8) * 2^(ex - 7); 0x7F / 0xFF give +-480 (the formula, not the NaN of e4m3fn).
// Built from the bit pattern: exponent field ex + 120, mantissa mt in the top 3 bits.
__device__ __forceinline__ float fp8_e4m3(uint32_t c) {
  const uint32_t ex = (c >> 3) & 15u, mt = c & 7u;
  const float mag = ex ? __uint_as_float(((ex + 120u) << 23) | (mt << 20)) : (float)mt * 0.001953125f;
  return (c & 128u) ? -mag : mag;
}

// float -> bfloat16 bits, round to nearest even (NaN -> 0x7FC0).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// float -> fp16 bits, round to nearest even (the conversion instruction rounds to nearest even).
// The empty asm keeps the compiler from folding a preceding multiply into the conversion as
// v_fma_mixlo_f16 a, b, 0: adding +0 turns a -0 product into +0.
__device__ __forceinline__ uint32_t f16_bits(float f) {
  asm volatile("" : "+v"(f));
  _Float16 h = (_Float16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// Round a float to the storage dtype's bits (BH_HEX_BF16 / BH_HEX_F16).
template <int DT>
__device__ __forceinline__ uint32_t to_bits(float f) {
  if constexpr (DT == BH_HEX_BF16) return bf16_bits(f);
  else return f16_bits(f);
}
template <int DT>
__device__ __forceinline__ float from_bits(uint32_t b) {
  if constexpr (DT == BH_HEX_BF16) return bf16_to_f32(b);
  else return f16_to_f32(b);
}

// ----------------------------------------------------------------------------------- matrix cores

// D = A * B + C on a 16x16x32 tile. Lane l supplies A[l % 16][8 (l / 16) + 0..7] and
// B[8 (l / 16) + 0..7][l % 16] (8 consecutive-K values in 4 dwords, low half first);
// D[4 (l / 16) + r][l % 16] lands in register r.
template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == BH_HEX_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
}

// Cross-row exchanges of a wave (rows = 16 lanes):
//   swap32(x, y): x[lanes 32..63] <-> y[lanes 0..31]
//   swap16(x, y): x[odd rows]     <-> y[even rows]
__device__ __forceinline__ void swap32(uint32_t& x, uint32_t& y) {
  auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  x = r[0];
  y = r[1];
}
__device__ __forceinline__ void swap16(uint32_t& x, uint32_t& y) {
  auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
  x = r[0];
  y = r[1];
}

// 4x4 transpose across the four rows of a wave: on entry row g of r[j] holds item (g, j); on
// exit row g of r[q] holds item (q, g).
__device__ __forceinline__ void transpose_rows4(uint32_t r[4]) {
  swap32(r[0], r[2]);
  swap32(r[1], r[3]);
  swap16(r[0], r[1]);
  swap16(r[2], r[3]);
}

// ----------------------------------------------------------------------------------- workgroup helpers

constexpr int kScanThreads = 1024;                 // workgroup size of the scan below
constexpr int kScanWaves = kScanThreads / kWave;

// Inclusive prefix sum over a 1024-thread workgroup of one value per thread; wsum is kScanWaves
// ints of LDS. Every thread of the workgroup must call it (it holds three barriers).
__device__ __forceinline__ int block_incl_scan(int v, int* wsum) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  if (lane == kWave - 1) wsum[w] = v;
  __syncthreads();
  if (w == 0) {
    int s = lane < kScanWaves ? wsum[lane] : 0;
#pragma unroll
    for (int d = 1; d < kScanWaves; d <<= 1) {
      const int o = __shfl_up(s, d, kWave);
      if (lane >= d) s += o;
    }
    if (lane < kScanWaves) wsum[lane] = s;
  }
  __syncthreads();
  const int r = v + (w ? wsum[w - 1] : 0);
  __syncthreads();
  return r;
}

// The lanes of a wave holding the same key as this lane (one ballot per bit of the key's
// nbits bits, so the cost does not depend on how many distinct keys the wave holds).
__device__ __forceinline__ uint64_t match_key(int key, int nbits) {
  uint64_t same = ~0ull;
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (key >> b) & 1;
    const uint64_t bal = __ballot(bit);
    same &= bit ? bal : ~bal;
  }
  return same;
}

// ----------------------------------------------------------------------------------- host side

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace bh
