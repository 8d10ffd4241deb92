// Pieces shared by the fused HEX expert kernels: the launch arguments, fp8 scale decoding,
// pair-table operand lookup, and raw buffer loads.
#pragma once

#include "hex_common.h"

namespace bh {

int check_proj(const bh_hex_proj* w, int64_t n_in, const char* who, int* block);

struct MoeArgs {
  const uint16_t* x;     // activations [rows, K] (bf16/f16 bits)
  int64_t s_xm;
  void* out;             // GLU: act [slots, N] (activation dtype); down: y [slots, N] float
  int64_t s_om;          //   (or, with y16, y in the activation dtype)
  bh_hex_proj w0, w1;    // gate, up (GLU) or down (w0 only)
  const int32_t* sid;     // the slot plan (align's outputs), unless ids is set
  const int32_t* eid;
  const int32_t* npp;
  const void* ids;        // routing ids [num_slots] (I32 or I64): the kernel sorts them itself
  int32_t ids_i64;
  const int32_t* lookup;
  const float* topk_w;
  int64_t num_slots;
  int32_t n_experts;
  int32_t a_div;
  int32_t N, K;
  int32_t y16;           // down: y is in the activation dtype (else float32)
  int32_t scale_words;   // block_scale rows allow one load of a unit's scales (8 or 2 bytes)
                         // (host only: it selects the whole-unit kernel variant)
  float* part;           // workspace: partial sums of items split between workgroups
  int32_t* counters;     // workspace: arrivals per split item (64 bytes apart), zero between calls
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

// The same without a branch (byte 0 of b): the instruction, then +-480 for 0x7F / 0xFF.
__device__ __forceinline__ float fp8x1_nb(uint32_t b) {
  const float v = __builtin_amdgcn_cvt_f32_fp8((int)b, 0);
  return (b & 0x7Fu) == 0x7Fu ? ((b & 0x80u) ? -480.f : 480.f) : v;
}
__device__ __forceinline__ void fp8x4_nb(uint32_t w, float f[4]) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  const float v[4] = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t b = (w >> (8 * j)) & 0xFFu;
    f[j] = (b & 0x7Fu) == 0x7Fu ? ((b & 0x80u) ? -480.f : 480.f) : v[j];
  }
}

// Eight operands (two per dword, K order) for the codes of one 24/32-bit field, from a pair
// table in LDS: entry p holds (level[p & (L-1)], level[p >> bits]) in the activation dtype,
// one copy per lane slot, at byte (p << 8) | cb.
// ES = log2 of an entry's bytes (8: 64 copies; 7: 32 copies, 3-bit tables only).
template <int BITS, int ES = 8>
__device__ __forceinline__ u32x4 lookup8(uint32_t f, uint32_t cb, const uint32_t* tab) {
  static_assert(ES == 8 || (BITS == 3 && ES == 7), "4-bit tables have 64 copies");
  const char* base = reinterpret_cast<const char*>(tab);
  u32x4 b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t addr;
    if constexpr (BITS == 4) {
      addr = __builtin_amdgcn_perm(f, cb, 0x0C0C0000u | ((4u + j) << 8));  // byte j << 8 | cb
    } else {
      // ((f >> 6 j) & 63) << ES | cb as one shift and one v_and_or_b32 (the compiler's own
      // form is a shift, a mask and an add)
      const int d = ES - 6 * j;
      const uint32_t sh = d >= 0 ? f << d : f >> -d;
      asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(addr) : "v"(sh), "s"(63u << ES), "v"(cb));
    }
    b[j] = *reinterpret_cast<const uint32_t*>(base + addr);
  }
  return b;
}

// The packed words of a lane's 32-input block (four 32-bit words at 4 bits, three at 3 bits)
// as four fields of 8 codes, transposed across the wave's rows so that field q of lane
// (row ln, group lg) holds codes 8 lg .. 8 lg + 7 of block q of row ln: the operand the
// 16x16x32 MFMA takes from that lane for k-slice q.
template <int BITS, typename W>
__device__ __forceinline__ void fields(const W& w, uint32_t r[4]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = w[j];
  } else {   // the block's 96-bit stream as four 24-bit fields of 8 codes
    r[0] = w[0];
    r[1] = __builtin_amdgcn_alignbit(w[1], w[0], 24);
    r[2] = __builtin_amdgcn_alignbit(w[2], w[1], 16);
    r[3] = w[2] >> 8;
  }
  transpose_rows4(r);
}

constexpr int kRsrcWord3 = 0x00020000;   // raw buffer, 32-bit data format (gfx9 family)
constexpr int kCohere = 16;              // cache policy sc1: coherent across the device's L2s

// Buffer offsets are unsigned 32-bit values. kOOR is a byte offset past every resource: a load
// there returns zero and fetches nothing. Resources hold at most kMaxRecords bytes (the host
// entry points refuse larger tensors). A load's offset is the sum of at most two terms, each
// either kOOR or below kMaxRecords, plus an instruction offset below 4096: the sum stays below
// 2^32, and it is out of range whenever one term is kOOR. So nothing wraps.
constexpr uint32_t kOOR = 0x7FFF0000u;
constexpr uint32_t kMaxRecords = kOOR;
static_assert(kOOR >= kMaxRecords, "kOOR must lie past every resource");
static_assert(2ull * kOOR + 4096ull < (1ull << 32), "offset sums must not wrap");

// The signed VGPR offset the buffer builtins take, with the same 32 bits.
__device__ __forceinline__ int voff(uint32_t v) { return __builtin_bit_cast(int, v); }

// Raw buffer loads. They go through the compiler's buffer builtins, so the compiler tracks
// each one and waits for exactly the loads a use needs. The whole byte offset goes in the
// range-checked VGPR offset (soffset 0): an offset past the resource returns zero and fetches
// nothing.
template <int IMM>
__device__ __forceinline__ void ld_x4(u32x4& d, __amdgpu_buffer_rsrc_t r, uint32_t v) {
  d = __builtin_amdgcn_raw_buffer_load_b128(r, voff(v + IMM), 0, 0);
}
template <int IMM>
__device__ __forceinline__ void ld_x3(u32x3& d, __amdgpu_buffer_rsrc_t r, uint32_t v) {
  d = __builtin_amdgcn_raw_buffer_load_b96(r, voff(v + IMM), 0, 0);
}
template <int IMM>
__device__ __forceinline__ void ld_x2(u32x2& d, __amdgpu_buffer_rsrc_t r, uint32_t v) {
  d = __builtin_amdgcn_raw_buffer_load_b64(r, voff(v + IMM), 0, 0);
}
template <int IMM>
__device__ __forceinline__ void ld_x1(uint32_t& d, __amdgpu_buffer_rsrc_t r, uint32_t v) {
  d = __builtin_amdgcn_raw_buffer_load_b32(r, voff(v + IMM), 0, 0);
}
template <int IMM>
__device__ __forceinline__ void ld_u16(uint32_t& d, __amdgpu_buffer_rsrc_t r, uint32_t v) {
  d = __builtin_amdgcn_raw_buffer_load_b16(r, voff(v + IMM), 0, 0);
}
template <int IMM>
__device__ __forceinline__ void ld_u8(uint32_t& d, __amdgpu_buffer_rsrc_t r, uint32_t v) {
  d = __builtin_amdgcn_raw_buffer_load_b8(r, voff(v + IMM), 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(bytes > (int64_t)kMaxRecords ? (int64_t)kMaxRecords : bytes),
                                           kRsrcWord3);
}

// Brings every 64-byte line of a kernel's argument block (Args, passed by value as its first
// argument) into the scalar cache together, at kernel entry. The compiler loads an argument field
// where it is first used, each new line behind its own wait (an L2 round trip of a few hundred
// cycles, more while the weight stream loads the memory system); later loads of cached lines
// return in tens of cycles. (Measured on one box: config 2, T=16, 64.4 -> 63.0 us per layer in
// the decode kernels; 12.0 -> 12.6 us at T=1 in the matrix-vector kernels, whose short prologue
// then waits for lines it would not have needed yet, so those do not call it; no change in the
// prefill kernels.)
template <typename Args>
__device__ __forceinline__ void touch_args() {
  constexpr int kLines = (int)((sizeof(Args) + 63) / 64);
  const __attribute__((address_space(4))) uint32_t* k =
      (const __attribute__((address_space(4))) uint32_t*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t v[kLines];
#pragma unroll
  for (int i = 0; i < kLines; ++i) v[i] = k[16 * i];
#pragma unroll
  for (int i = 0; i < kLines; ++i) asm volatile("" ::"s"(v[i]));
}

// Host side.
int device_cus();
constexpr int kGemmMt = 8;   // block_m / 16 of the prefill kernels (128-slot blocks)
// Checks one projection for the fused kernels: scale blocks of 32 or 128 inputs (*sb = B / 32,
// equal to a nonzero *sb on entry), 16-byte aligned 4-bit rows, each expert's matrix within one
// buffer resource; clears *words when the scale rows do not allow one load of a unit's scales.
int proj_setup(const char* who, const bh_hex_proj* w, int bits, int64_t n_out, int64_t n_in, int* sb, int* words);
// Launches the prefill kernels for a plan of 128-slot blocks (no workspace).
int gemm_run(const char* who, bool glu, int bits, int adt, int sb, const MoeArgs& a, int64_t num_blocks,
             hipStream_t stream);
inline bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

}  // namespace bh
