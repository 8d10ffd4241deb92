// The GPTQ column sweep of the HEX producer, rounding onto each expert's level table.
//
// Replaces the torch sweep of reaper/gpu_perf/gptq.py:62-83 (_solve: columns in order, each
// rounded to the nearest level of its scaled table, its error divided by the factor's diagonal
// and pushed onto the rest of its 128-column block at once, and onto the later columns when the
// block ends) and the table indices of harness/blackhole_pipeline/pack.py:53-62 (table_indices)
// for device tensors.
//
// Each weight row's sweep depends only on that row and the factor U, so one lane owns one row.
// The row's current block lives in LDS column-major (lane r's value of column c at [c][r]: lanes
// never share a bank), and the block's errors replace its columns as they are finalised. The
// factor's values are the same for every lane and come in through scalar loads. The arithmetic
// is the reference's on the CPU, operation for operation: IEEE divides, a product and a
// difference rounded separately in the block update (no contraction), and the later columns'
// update as one fused multiply-add chain over the block's errors in column order, which is how
// the CPU's matrix product accumulates it. So the outputs equal the reference's bit for bit on
// the same inputs.
#include <string>

#include "hex_common.h"

namespace bh {

constexpr int kGqRows = kWave;          // rows of a workgroup: one per lane
constexpr int kGqBlock = 128;           // most columns of one sweep block (the LDS block)
constexpr int kGqChunk = 16;            // later columns updated together

struct GptqArgs {
  float* w;                 // [n, out, in] working weights (the sweep updates them)
  const float* u;           // [n, in, in] upper factor of the damped inverse Hessian
  const float* levels;      // [n, L] sorted
  const float* scale;       // [n, out, in / sblock] dequant scale per scale block
  const uint8_t* dead;      // [n, in] or null
  float* q;                 // [n, out, in] rounded weights
  uint8_t* codes;           // [n, out, in] table indices of q
  int32_t out, in, sblock, block;
};

// Index of the nearest level of v: the number of midpoints below v (a left search).
template <int L>
__device__ __forceinline__ int nearest(float v, const float (&mid)[L - 1]) {
  int i = 0;
#pragma unroll
  for (int m = 0; m < L - 1; ++m) i += mid[m] < v ? 1 : 0;
  return i;
}

// Level i, from the lane that holds it (lane m holds level m in levv).
__device__ __forceinline__ float level_at(int i, float levv) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(i * 4, __builtin_bit_cast(int, levv)));
}

template <int L>
__global__ __launch_bounds__(kGqRows) void gptq_sweep_kernel(GptqArgs a) {
#pragma clang fp contract(off)
  __shared__ float lw[kGqBlock][kGqRows];
  const int lane = threadIdx.x;
  const int e = blockIdx.y;
  const int r = blockIdx.x * kGqRows + lane;
  const bool row = r < a.out;
  const int64_t in = a.in;
  float* wr = a.w + ((int64_t)e * a.out + (row ? r : 0)) * in;
  const float* ue = a.u + (int64_t)e * in * in;
  const float* sr = a.scale + ((int64_t)e * a.out + (row ? r : 0)) * (in / a.sblock);
  float* qr = a.q + ((int64_t)e * a.out + (row ? r : 0)) * in;
  const float* le = a.levels + (int64_t)e * L;
  const float levv = lane < L ? le[lane] : 0.f;
  float mid[L - 1];                     // the midpoints, as the reference forms them: (a + b) / 2
#pragma unroll
  for (int m = 0; m < L - 1; ++m) mid[m] = (le[m + 1] + le[m]) / 2.0f;
  for (int b0 = 0; b0 < a.in; b0 += a.block) {
    const int cols = min(a.block, a.in - b0);
    for (int c = 0; c < cols; ++c) lw[c][lane] = row ? wr[b0 + c] : 0.f;
    for (int j = 0; j < cols; ++j) {
      const float x = lw[j][lane];
      const float s = sr[(b0 + j) / a.sblock];
      const float v = fminf(fmaxf(x / s, -1.0f), 1.0f);
      const float qv = level_at(nearest<L>(v, mid), levv) * s;
      if (row) qr[b0 + j] = qv;
      const float* uj = ue + (int64_t)(b0 + j) * in + b0;
      const float err = (x - qv) / uj[j];
      lw[j][lane] = err;                 // column j is final: its slot keeps the error
      for (int c = j + 1; c < cols; ++c) lw[c][lane] = lw[c][lane] - err * uj[c];
    }
    // the later columns: w -= (errors of the block) . U[block rows, column], chained in order
    for (int c0 = b0 + cols; c0 < a.in; c0 += kGqChunk) {
      float acc[kGqChunk];
#pragma unroll
      for (int i = 0; i < kGqChunk; ++i) acc[i] = 0.f;
      const int valid = min(kGqChunk, a.in - c0);
      for (int k = 0; k < cols; ++k) {
        const float ek = lw[k][lane];
        const float* uk = ue + (int64_t)(b0 + k) * in + c0;
        if (valid == kGqChunk) {
#pragma unroll
          for (int i = 0; i < kGqChunk; ++i) acc[i] = __builtin_fmaf(ek, uk[i], acc[i]);
        } else {
#pragma unroll
          for (int i = 0; i < kGqChunk; ++i)
            if (i < valid) acc[i] = __builtin_fmaf(ek, uk[i], acc[i]);
        }
      }
      if (row) {
#pragma unroll
        for (int i = 0; i < kGqChunk; ++i)
          if (i < valid) wr[c0 + i] = wr[c0 + i] - acc[i];
      }
    }
  }
  // dead columns zeroed (q times 0, as the reference's mask product), then the table indices
  if (!row) return;
  uint8_t* cr = a.codes + ((int64_t)e * a.out + r) * in;
  for (int c = 0; c < a.in; ++c) {
    float qv = qr[c];
    if (a.dead) qv = qv * (a.dead[(int64_t)e * in + c] ? 0.0f : 1.0f);
    qr[c] = qv;
    const float s = sr[c / a.sblock];
    cr[c] = (uint8_t)nearest<L>(fminf(fmaxf(qv / s, -1.0f), 1.0f), mid);
  }
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_gptq_sweep(float* w, const float* u, const float* levels, int32_t n_levels, const float* scale,
                                 int32_t scale_block, const uint8_t* dead, int64_t n, int64_t out, int64_t in,
                                 int32_t block, float* q, uint8_t* codes, void* stream) {
  const char* who = "bh_hex_gptq_sweep";
  if (n_levels != 8 && n_levels != 16) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": 8 or 16 levels");
  if (n < 0 || out < 0 || in <= 0 || block <= 0 || block > kGqBlock || scale_block <= 0 || in % scale_block)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes (block 1..128, in a multiple of scale_block)");
  if (n > 65535 || out > (int64_t)65535 * kGqRows || in > (1 << 24))
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": too many experts, rows or columns");
  if (n == 0 || out == 0) return BH_HEX_OK;
  if (!w || !u || !levels || !scale || !q || !codes) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  GptqArgs a{w, u, levels, scale, dead, q, codes, (int32_t)out, (int32_t)in, scale_block, block};
  const dim3 grid((unsigned)cdiv(out, kGqRows), (unsigned)n);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n_levels == 16) hipLaunchKernelGGL(gptq_sweep_kernel<16>, grid, dim3(kGqRows), 0, st, a);
  else hipLaunchKernelGGL(gptq_sweep_kernel<8>, grid, dim3(kGqRows), 0, st, a);
  return check_launch(who);
}
