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
// factor's values are the same for every lane: the block's diagonal part is staged in LDS once
// per block, and the later columns' part goes through LDS 16 columns at a time, the next chunk
// (with the rows' weights it updates) requested while the current one is applied. The arithmetic
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
constexpr int kGqChunkLoads = kGqBlock * kGqChunk / kGqRows;   // factor values per lane per chunk
constexpr int kGqScales = kGqBlock / 32 + 1;                    // a block's scale blocks (at least 32 inputs)

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

struct GqLds {
  float lw[kGqBlock][kGqRows];              // the rows' current block, column-major
  float ub[kGqBlock][kGqBlock];             // U[b0 + k][b0 + c] of the block
  float uc[2][kGqBlock][kGqChunk];          // U[b0 + k][c0 + i] of a later chunk, two chunks
  float ls[kGqScales][kGqRows];             // the rows' scales of the block's scale blocks
};

template <int L>
__global__ __launch_bounds__(kGqRows) void gptq_sweep_kernel(GptqArgs a) {
#pragma clang fp contract(off)
  __shared__ GqLds sm;
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
  // factor values of one later chunk for this lane: entry t is U[b0 + k][c0 + i] with
  // (k, i) = ((lane + 64 t) / 16, (lane + 64 t) % 16); nothing past the block or the matrix
  auto chunk_load = [&](float (&v)[kGqChunkLoads], int b0, int cols, int c0) {
#pragma unroll
    for (int t = 0; t < kGqChunkLoads; ++t) {
      const int x = lane + kGqRows * t, k = x / kGqChunk, i = x % kGqChunk;
      v[t] = (k < cols && c0 + i < a.in) ? ue[(int64_t)(b0 + k) * in + c0 + i] : 0.f;
    }
  };
  auto chunk_store = [&](const float (&v)[kGqChunkLoads], int buf) {
#pragma unroll
    for (int t = 0; t < kGqChunkLoads; ++t) {
      const int x = lane + kGqRows * t;
      sm.uc[buf][x / kGqChunk][x % kGqChunk] = v[t];
    }
  };
  // the row's weights of a later chunk
  auto row_load = [&](float (&v)[kGqChunk], int c0) {
#pragma unroll
    for (int i = 0; i < kGqChunk; ++i) v[i] = (row && c0 + i < a.in) ? wr[c0 + i] : 0.f;
  };
  for (int b0 = 0; b0 < a.in; b0 += a.block) {
    const int cols = min(a.block, a.in - b0);
    // the block: the rows' weights, the factor's diagonal part and the rows' scales, all
    // requested before any is stored
    for (int c = 0; c < cols; c += kGqChunk) {
      float v[kGqChunk];
#pragma unroll
      for (int i = 0; i < kGqChunk; ++i) v[i] = (row && c + i < cols) ? wr[b0 + c + i] : 0.f;
#pragma unroll
      for (int i = 0; i < kGqChunk; ++i)
        if (c + i < cols) sm.lw[c + i][lane] = v[i];
    }
    for (int x0 = 0; x0 < cols * cols; x0 += kGqRows * kGqChunk) {
      float v[kGqChunk];
#pragma unroll
      for (int t = 0; t < kGqChunk; ++t) {
        const int x = x0 + lane + kGqRows * t, k = x / cols, c = x % cols;
        v[t] = x < cols * cols ? ue[(int64_t)(b0 + k) * in + b0 + c] : 0.f;
      }
#pragma unroll
      for (int t = 0; t < kGqChunk; ++t) {
        const int x = x0 + lane + kGqRows * t;
        if (x < cols * cols) sm.ub[x / cols][x % cols] = v[t];
      }
    }
    const int sb0 = b0 / a.sblock, nsb = (b0 + cols - 1) / a.sblock - sb0 + 1;   // nsb <= kGqScales
    for (int q = 0; q < nsb; ++q) sm.ls[q][lane] = row ? sr[sb0 + q] : 1.f;
    __syncthreads();
    for (int j = 0; j < cols; ++j) {
      const float x = sm.lw[j][lane];
      const float s = sm.ls[(b0 + j) / a.sblock - sb0][lane];
      const float v = fminf(fmaxf(x / s, -1.0f), 1.0f);
      const float qv = level_at(nearest<L>(v, mid), levv) * s;
      if (row) qr[b0 + j] = qv;
      const float err = (x - qv) / sm.ub[j][j];
      sm.lw[j][lane] = err;              // column j is final: its slot keeps the error
      for (int c = j + 1; c < cols; ++c) sm.lw[c][lane] = sm.lw[c][lane] - err * sm.ub[j][c];
    }
    // the later columns: w -= (errors of the block) . U[block rows, column], chained in order;
    // chunk c0's factor values and weights were requested while the previous chunk was applied
    const int c_first = b0 + cols;
    if (c_first < a.in) {
      float fv[kGqChunkLoads], wv[kGqChunk];
      chunk_load(fv, b0, cols, c_first);
      row_load(wv, c_first);
      int buf = 0;
      for (int c0 = c_first; c0 < a.in; c0 += kGqChunk) {
        chunk_store(fv, buf);
        float wc[kGqChunk];
#pragma unroll
        for (int i = 0; i < kGqChunk; ++i) wc[i] = wv[i];
        __syncthreads();                 // this chunk's factor values are in LDS
        if (c0 + kGqChunk < a.in) {      // (uniform) the next chunk, in flight during this one
          chunk_load(fv, b0, cols, c0 + kGqChunk);
          row_load(wv, c0 + kGqChunk);
        }
        float acc[kGqChunk];
#pragma unroll
        for (int i = 0; i < kGqChunk; ++i) acc[i] = 0.f;
        for (int k = 0; k < cols; ++k) {
          const float ek = sm.lw[k][lane];
#pragma unroll
          for (int i = 0; i < kGqChunk; ++i) acc[i] = __builtin_fmaf(ek, sm.uc[buf][k][i], acc[i]);
        }
        if (row) {
          const int valid = min(kGqChunk, a.in - c0);
#pragma unroll
          for (int i = 0; i < kGqChunk; ++i)
            if (i < valid) wr[c0 + i] = wc[i] - acc[i];
        }
        buf ^= 1;
      }
    }
    __syncthreads();                     // the block's LDS is read out before the next block's
  }
  // dead columns zeroed (q times 0, as the reference's mask product), then the table indices;
  // 16 columns' loads at a time
  if (!row) return;
  uint8_t* cr = a.codes + ((int64_t)e * a.out + r) * in;
  for (int c0 = 0; c0 < a.in; c0 += kGqChunk) {
    float qv[kGqChunk], sv[kGqChunk];
    bool dd[kGqChunk];
#pragma unroll
    for (int i = 0; i < kGqChunk; ++i) {
      const int c = min(c0 + i, a.in - 1);
      qv[i] = qr[c];
      sv[i] = sr[c / a.sblock];
      dd[i] = a.dead ? a.dead[(int64_t)e * in + c] != 0 : false;
    }
#pragma unroll
    for (int i = 0; i < kGqChunk; ++i) {
      if (c0 + i < a.in) {
        const float q = qv[i] * (dd[i] ? 0.0f : 1.0f);
        qr[c0 + i] = a.dead ? q : qv[i];
        cr[c0 + i] = (uint8_t)nearest<L>(fminf(fmaxf((a.dead ? q : qv[i]) / sv[i], -1.0f), 1.0f), mid);
      }
    }
  }
}

// ----------------------------------------------------------------------------------- header

constexpr int kHdThreads = 1024;
constexpr float kFp8Max = 448.0f;

// v in [0, 448] rounded to the nearest fp8 e4m3fn value (ties to even): a multiple of the value's
// fp8 spacing, 2^(e - 3) for exponents e >= -6 and 2^-9 below (the subnormals). Scaling by a power
// of two is exact, so the one rounding is the round-to-nearest-even of v / spacing.
__device__ __forceinline__ float fp8_round(float v) {
  const int ex = (int)((__float_as_uint(v) >> 23) & 0xFFu) - 127;
  const int sp = (ex < -6 ? -6 : ex) - 3;
  return __builtin_ldexpf(__builtin_rintf(__builtin_ldexpf(v, -sp)), sp);
}

// The e4m3fn code of an fp8 value q in [0, 448] (as fp8_round returns).
__device__ __forceinline__ uint32_t fp8_code(float q) {
  if (q == 0.0f) return 0u;
  const uint32_t b = __float_as_uint(q);
  const int ex = (int)((b >> 23) & 0xFFu) - 127;
  if (ex < -6) return (uint32_t)__builtin_rintf(__builtin_ldexpf(q, 9));     // subnormal: q / 2^-9
  return ((uint32_t)(ex + 7) << 3) | ((b >> 20) & 7u);
}

// One workgroup per expert: es = max(max|w| / 448, 1e-30); per block of `block` inputs the
// dequant scale fp8(min(amax / es, 448)) * es (1 where that is 0), its fp8 code of
// min(scale / es, 448), the values clamp(w / scale, -1, 1), and (col_weight given) the k-means
// weights col_weight[col] * scale^2 (reaper/gpu_perf/headers.py:39-51, 96-98;
// harness/blackhole_pipeline/pack.py:77-86).
__global__ __launch_bounds__(kHdThreads) void block_header_kernel(const float* w, int64_t out, int64_t in, int block,
                                                                  const float* col_weight, float* xn, float* scale,
                                                                  uint8_t* codes, float* wt, float* es_out) {
#pragma clang fp contract(off)
  __shared__ float red[kHdThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t e = blockIdx.x, m = out * in, nb = m / block;
  const float* we = w + e * m;
  float mx = 0.f;
  for (int64_t i = tid; i < m; i += kHdThreads) mx = fmaxf(mx, fabsf(we[i]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  float top = 0.f;
#pragma unroll
  for (int i = 0; i < kHdThreads / kWave; ++i) top = fmaxf(top, red[i]);
  const float es = fmaxf(top / kFp8Max, 1e-30f);
  if (tid == 0) es_out[e] = es;
  for (int64_t bk = tid; bk < nb; bk += kHdThreads) {
    const float* x = we + bk * block;
    float amax = 0.f;
    for (int i = 0; i < block; ++i) amax = fmaxf(amax, fabsf(x[i]));
    float blk = fp8_round(fminf(amax / es, kFp8Max)) * es;
    if (!(blk > 0.0f)) blk = 1.0f;
    scale[e * nb + bk] = blk;
    if (codes) codes[e * nb + bk] = (uint8_t)fp8_code(fp8_round(fminf(blk / es, kFp8Max)));
    const int64_t col0 = (bk * block) % in;
    const float b2 = blk * blk;
    for (int i = 0; i < block; ++i) {
      if (xn) xn[e * m + bk * block + i] = fminf(fmaxf(x[i] / blk, -1.0f), 1.0f);
      if (wt) wt[e * m + bk * block + i] = col_weight[e * in + col0 + i] * b2;
    }
  }
}

// ----------------------------------------------------------------------------------- k-means

// One wave per expert, lane l owning level l: the start is the linear-interpolation quantile
// lo + w (hi - lo) of the sorted sample (ATen's form: an FMA on the end nearer the weight), then
// `iters` Lloyd rounds: every value goes to the level of its left midpoint search, each level's
// sums of x*w and w run over its values in sample order (as the CPU's scatter_add), the level
// moves to num / max(den, 1e-30) where den > 0, and the levels are sorted
// (reaper/gpu_perf/headers.py:66-83).
template <int L>
__global__ __launch_bounds__(kWave) void fit_levels_kernel(const float* xs, const float* ws, int64_t S,
                                                           const float* q_lo, const float* q_hi, const float* q_w,
                                                           int iters, float* levels) {
#pragma clang fp contract(off)
  __shared__ float srt[L];
  const int lane = threadIdx.x;
  const int64_t e = blockIdx.x;
  const float* x = xs + e * S;
  const float* wv = ws + e * S;
  float lev = 0.f;
  if (lane < L) {
    const float lo = q_lo[e * L + lane], hi = q_hi[e * L + lane], wq = q_w[lane];
    const float d = hi - lo;
    lev = fabsf(wq) < 0.5f ? __builtin_fmaf(wq, d, lo) : __builtin_fmaf(wq - 1.0f, d, hi);
  }
  for (int it = 0; it < iters; ++it) {
    float mid[L - 1];
#pragma unroll
    for (int mi = 0; mi < L - 1; ++mi) {
      const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lev), mi + 1));
      const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lev), mi));
      mid[mi] = (a + b) / 2.0f;
    }
    float num = 0.f, den = 0.f;
    for (int64_t i = 0; i < S; ++i) {
      const float xi = x[i], wi = wv[i];
      int a = 0;
#pragma unroll
      for (int mi = 0; mi < L - 1; ++mi) a += mid[mi] < xi ? 1 : 0;
      if (a == lane) {
        num = num + xi * wi;
        den = den + wi;
      }
    }
    if (lane < L && den > 0.0f) lev = num / fmaxf(den, 1e-30f);
    // sort the L levels: lane l counts the levels below its own (ties by lane), then stores there
    int rank = 0;
#pragma unroll
    for (int mi = 0; mi < L; ++mi) {
      const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lev), mi));
      rank += (o < lev || (o == lev && mi < lane)) ? 1 : 0;
    }
    if (lane < L) srt[rank] = lev;
    __syncthreads();
    if (lane < L) lev = srt[lane];
    __syncthreads();
  }
  if (lane < L) levels[e * L + lane] = lev;
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_block_header(const float* w, int64_t n, int64_t out, int64_t in, int32_t block,
                                   const float* col_weight, float* xn, float* scale, uint8_t* codes, float* wt,
                                   float* expert_scale, void* stream) {
  const char* who = "bh_hex_block_header";
  if (n < 0 || out <= 0 || in <= 0 || block <= 0 || in % block)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes (in a multiple of block)");
  if (n == 0) return BH_HEX_OK;
  if (!w || !scale || !expert_scale || (wt && !col_weight)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  hipLaunchKernelGGL(block_header_kernel, dim3((unsigned)n), dim3(kHdThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     w, out, in, block, col_weight, xn, scale, codes, wt, expert_scale);
  return check_launch(who);
}

extern "C" int bh_hex_fit_levels(const float* xs, const float* ws, int64_t n, int64_t S, int32_t n_levels,
                                 const float* q_lo, const float* q_hi, const float* q_w, int32_t iters, float* levels,
                                 void* stream) {
  const char* who = "bh_hex_fit_levels";
  if (n_levels != 8 && n_levels != 16) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": 8 or 16 levels");
  if (n < 0 || S <= 0 || iters < 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes");
  if (n == 0) return BH_HEX_OK;
  if (!xs || !ws || !q_lo || !q_hi || !q_w || !levels) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n_levels == 16)
    hipLaunchKernelGGL(fit_levels_kernel<16>, dim3((unsigned)n), dim3(kWave), 0, st, xs, ws, S, q_lo, q_hi, q_w, iters, levels);
  else
    hipLaunchKernelGGL(fit_levels_kernel<8>, dim3((unsigned)n), dim3(kWave), 0, st, xs, ws, S, q_lo, q_hi, q_w, iters, levels);
  return check_launch(who);
}

extern "C" int bh_hex_gptq_sweep(float* w, const float* u, const float* levels, int32_t n_levels, const float* scale,
                                 int32_t scale_block, const uint8_t* dead, int64_t n, int64_t out, int64_t in,
                                 int32_t block, float* q, uint8_t* codes, void* stream) {
  const char* who = "bh_hex_gptq_sweep";
  if (n_levels != 8 && n_levels != 16) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": 8 or 16 levels");
  if (n < 0 || out < 0 || in <= 0 || block <= 0 || block > kGqBlock || scale_block <= 0 || in % scale_block)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes (block 1..128, in a multiple of scale_block)");
  if (n > 65535 || out > (int64_t)65535 * kGqRows || in > (1 << 24))
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": too many experts, rows or columns");
  if (scale_block < 32)   // a block's scales are staged for at most kGqScales scale blocks
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": scale blocks of at least 32 inputs");
  if (n == 0 || out == 0) return BH_HEX_OK;
  if (!w || !u || !levels || !scale || !q || !codes) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  GptqArgs a{w, u, levels, scale, dead, q, codes, (int32_t)out, (int32_t)in, scale_block, block};
  const dim3 grid((unsigned)cdiv(out, kGqRows), (unsigned)n);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n_levels == 16) hipLaunchKernelGGL(gptq_sweep_kernel<16>, grid, dim3(kGqRows), 0, st, a);
  else hipLaunchKernelGGL(gptq_sweep_kernel<8>, grid, dim3(kGqRows), 0, st, a);
  return check_launch(who);
}
