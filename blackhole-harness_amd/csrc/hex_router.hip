// Expert routing in front of the HEX MoE layer: the reference's route_from_logits
// (reaper/reaper_pipeline/moe.py:141-168) as vLLM runs it before HexMoEMethod.apply.
//
//   bh_hex_route_topk    softmax top-k of router logits (the softmax branch), one wave per token
//   bh_hex_route_select  both branches: softmax, or sigmoid scores with an optional correction
//                        bias and group-limited choice; renormalisation; routed_scaling_factor
//   bh_hex_route_gemm    the router logits x @ W^T (the model's gate linear, on the matrix cores)
//                        and the choice, in one launch
//
// One wave chooses one token's experts: expert e's value sits in lane e % 64, register e / 64
// (up to 1024 experts). A choice round is a butterfly argmax over the wave (ties to the lower
// expert id); the group-limited choice stages the token's values in the wave's own LDS row so
// that lane q can take the two largest of group q.
//
// The router GEMM: one workgroup per 16 tokens x 16 experts, its four waves taking alternate
// 32-input steps of the hidden size (so a decode batch still spreads over E / 16 workgroups),
// v_mfma_f32_16x16x32 on operands loaded straight from HBM/L2 (x rows and router rows, 16 bytes
// per lane), the four partials added in wave order in LDS. The logits are rounded to the
// activation dtype (the gate linear's output dtype) and stored; the last workgroup of a token
// tile to finish (an arrival counter per tile) then chooses the tile's experts.
#include <string>

#include "hex_fused.h"

namespace bh {

// Device copy of bh_hex_routing.
struct Routing {
  int32_t sigmoid, renorm, n_group, topk_group;
  float scale;
  const float* bias;
};

constexpr int kRtPerLane = 16;                 // experts per lane: up to 1024
constexpr int kRtMaxExperts = kWave * kRtPerLane;

template <int LDT>
__device__ __forceinline__ float load_logit(const void* p, int64_t i) {
  if constexpr (LDT == BH_HEX_F32) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (LDT == BH_HEX_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  else return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// Wave argmax of (v, i) with the larger v, then the lower i; carries a payload p.
__device__ __forceinline__ void wave_argmax(float& v, int& i, float& p) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(v, m, kWave);
    const int oi = __shfl_xor(i, m, kWave);
    const float op = __shfl_xor(p, m, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
      p = op;
    }
  }
}

// The experts of token t, chosen by the calling wave (all 64 lanes). l[j]: the logit of expert
// lane + 64 j (ignored past E). gl: E floats of LDS owned by this wave (group-limited choice).
template <int IDT>
__device__ __forceinline__ void select_token(const float (&l)[kRtPerLane], int E, int k, const Routing& r, float* gl,
                                             float* topk_w, void* topk_ids, int64_t t) {
  const int lane = threadIdx.x & 63;
  float s[kRtPerLane], c[kRtPerLane];     // score (the weight source) and choice value
  if (r.sigmoid) {
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j) {
      const int e = lane + kWave * j;
      s[j] = e < E ? 1.0f / (1.0f + expf(-l[j])) : 0.f;
      c[j] = e < E ? s[j] + (r.bias ? r.bias[e] : 0.f) : -INFINITY;
    }
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j)
      if (lane + kWave * j < E) mx = fmaxf(mx, l[j]);
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j) {
      s[j] = lane + kWave * j < E ? expf(l[j] - mx) : 0.f;
      sum += s[j];
    }
    sum = wave_sum(sum);
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j) {
      const bool ok = lane + kWave * j < E;
      s[j] = ok ? s[j] / sum : 0.f;
      c[j] = ok ? s[j] : -INFINITY;
    }
  }
  if (r.sigmoid && r.n_group > 1) {
    // group q = experts [q G, (q + 1) G) scores the sum of its two largest choices; the
    // topk_group best groups stay, every other expert's choice becomes -inf
    const int G = E / r.n_group;
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j)
      if (lane + kWave * j < E) gl[lane + kWave * j] = c[j];
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    float gs = -INFINITY;
    if (lane < r.n_group) {
      float m1 = -INFINITY, m2 = -INFINITY;
      for (int i = 0; i < G; ++i) {
        const float v = gl[lane * G + i];
        if (v > m1) {
          m2 = m1;
          m1 = v;
        } else if (v > m2) {
          m2 = v;
        }
      }
      gs = m1 + m2;
    }
    uint64_t kept = 0;
    const int tg = r.topk_group > 0 ? r.topk_group : r.n_group;
    for (int q = 0; q < tg; ++q) {
      float bv = lane < r.n_group ? gs : -INFINITY, bp = 0.f;
      int bi = lane < r.n_group ? lane : 0x7FFFFFFF;
      wave_argmax(bv, bi, bp);
      kept |= 1ull << bi;               // (at most 64 groups: one bit each)
      if (lane == bi) gs = -INFINITY;   // a chosen group then loses to every finite group score
    }
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j) {
      const int e = lane + kWave * j;
      if (e < E && !((kept >> (e / G)) & 1ull)) c[j] = -INFINITY;
    }
  }
  uint32_t taken = 0;                     // bit j: expert lane + 64 j already chosen
  float wsel = 0.f, wsum = 0.f;
  int isel = 0;
  for (int rr = 0; rr < k; ++rr) {
    float bv = -INFINITY, bp = 0.f;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j) {
      const int e = lane + kWave * j;
      if (e < E && !((taken >> j) & 1u) && (c[j] > bv || (c[j] == bv && e < bi))) {
        bv = c[j];
        bi = e;
        bp = s[j];
      }
    }
    wave_argmax(bv, bi, bp);
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    wsum += bp;
    if (lane == rr) {
      wsel = bp;
      isel = bi;
    }
  }
  if (lane < k) {
    float w = wsel;
    if (r.renorm) w = r.sigmoid ? w / (wsum + 1e-20f) : w / wsum;
    w *= r.scale;
    topk_w[t * k + lane] = w;
    if constexpr (IDT == BH_HEX_I64) reinterpret_cast<int64_t*>(topk_ids)[t * k + lane] = isel;
    else reinterpret_cast<int32_t*>(topk_ids)[t * k + lane] = isel;
  }
}

// Choice from logits [T, E] (row stride s_lt): one wave per token, four tokens per workgroup.
template <int LDT, int IDT>
__global__ __launch_bounds__(256) void route_select_kernel(const void* __restrict__ logits, int64_t s_lt, int64_t T,
                                                           int32_t E, int32_t k, Routing r, float* __restrict__ topk_w,
                                                           void* __restrict__ topk_ids) {
  __shared__ float gl[4][kRtMaxExperts];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t >= T) return;                   // (no workgroup barrier follows)
  float l[kRtPerLane];
#pragma unroll
  for (int j = 0; j < kRtPerLane; ++j) {
    const int e = lane + kWave * j;
    l[j] = e < E ? load_logit<LDT>(logits, t * s_lt + e) : 0.f;
  }
  select_token<IDT>(l, E, k, r, gl[wave], topk_w, topk_ids, t);
}

// Router logits and choice. Workgroup (tile of 16 tokens, tile of 16 experts).
constexpr int kRtSteps = 8;            // 32-input steps whose loads a wave issues together
template <int ADT, int IDT>
__global__ __launch_bounds__(256) void route_gemm_kernel(const uint16_t* __restrict__ x, int64_t s_xm,
                                                         const uint16_t* __restrict__ wr, int64_t s_we, int32_t T,
                                                         int32_t H, int32_t E, int32_t k, Routing r,
                                                         float* __restrict__ logits, int64_t s_lt,
                                                         float* __restrict__ topk_w, void* __restrict__ topk_ids,
                                                         int32_t* __restrict__ counters) {
  __shared__ __align__(16) float red[4][kWave * 4];
  __shared__ float gl[4][kRtMaxExperts];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tt = blockIdx.x, et = blockIdx.y;
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, (int64_t)T * s_xm * 2);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wr, (int64_t)E * s_we * 2);
  // lane (row l % 16, k-group l / 16): A = token rows, B = router rows (16x16x32 operand layout)
  const int tok = tt * 16 + (lane & 15), ex = et * 16 + (lane & 15);
  const uint32_t xo = tok < T ? (uint32_t)(tok * s_xm * 2) + (uint32_t)(lane >> 4) * 16u : kOOR;
  const uint32_t wo = ex < E ? (uint32_t)(ex * s_we * 2) + (uint32_t)(lane >> 4) * 16u : kOOR;
  const int nsteps = H / 32;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < nsteps; s0 += 4 * kRtSteps) {
    u32x4 a[kRtSteps], b[kRtSteps];
#pragma unroll
    for (int i = 0; i < kRtSteps; ++i) {
      const int s = s0 + 4 * i;
      const uint32_t off = s < nsteps ? (uint32_t)s * 64u : kOOR;
      a[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, voff(s < nsteps ? xo + off : kOOR), 0, 0);
      b[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, voff(s < nsteps ? wo + off : kOOR), 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kRtSteps; ++i) acc = mfma16x16x32<ADT>(a[i], b[i], acc);
  }
  *reinterpret_cast<f32x4*>(&red[wave][lane * 4]) = acc;
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(logits, (int64_t)T * s_lt * 4);
  if (wave == 0) {
    const f32x4 v = ((*reinterpret_cast<const f32x4*>(&red[0][lane * 4]) + *reinterpret_cast<const f32x4*>(&red[1][lane * 4])) +
                     *reinterpret_cast<const f32x4*>(&red[2][lane * 4])) + *reinterpret_cast<const f32x4*>(&red[3][lane * 4]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = tt * 16 + 4 * (lane >> 4) + q, e = et * 16 + (lane & 15);
      if (t < T && e < E) {           // rounded as the gate linear's output dtype, kept as float
        const float lg = from_bits<ADT>(to_bits<ADT>(v[q]));
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, lg), rl,
                                              voff((uint32_t)((int64_t)t * s_lt + e) * 4u), 0, kCohere);
      }
    }
  }
  // the last workgroup of this token tile to arrive chooses its tokens' experts
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(counters + tt * 16, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == (int)gridDim.y - 1;
    if (last) __hip_atomic_store(counters + tt * 16, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  for (int i = 0; i < 4; ++i) {
    const int t = tt * 16 + wave * 4 + i;
    if (t >= T) break;                 // (wave-uniform; no workgroup barrier follows)
    float l[kRtPerLane];
#pragma unroll
    for (int j = 0; j < kRtPerLane; ++j) {
      const int e = lane + kWave * j;
      l[j] = e < E ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                   rl, voff((uint32_t)((int64_t)t * s_lt + e) * 4u), 0, kCohere))
                   : 0.f;
    }
    select_token<IDT>(l, E, k, r, gl[wave], topk_w, topk_ids, t);
  }
}

// ----------------------------------------------------------------------------------- host side

static int check_routing(const char* who, int32_t E, int32_t k, const bh_hex_routing* in, Routing* out) {
  if (E <= 0 || E > kRtMaxExperts)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": experts must be in 1.." + std::to_string(kRtMaxExperts));
  if (k <= 0 || k > E || k > kWave) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": k must be in 1..min(E, 64)");
  Routing r{0, 1, 1, 0, 1.0f, nullptr};
  if (in) {
    if (in->scoring != BH_HEX_SCORE_SOFTMAX && in->scoring != BH_HEX_SCORE_SIGMOID)
      return fail(BH_HEX_ERR_VALUE, std::string(who) + ": scoring must be softmax or sigmoid");
    // a correction bias selects the sigmoid branch whatever the scoring (moe.py:148)
    r.sigmoid = in->scoring == BH_HEX_SCORE_SIGMOID || in->correction_bias != nullptr;
    r.renorm = in->renormalize != 0;
    r.n_group = in->n_group;
    r.topk_group = in->topk_group;
    r.scale = in->routed_scaling_factor;
    r.bias = in->correction_bias;
    if (r.n_group < 1 || r.n_group > kWave || E % r.n_group || (r.n_group > 1 && E / r.n_group < 2))
      return fail(BH_HEX_ERR_VALUE, std::string(who) + ": n_group must divide the experts into groups of at least "
                                                       "two, at most 64 groups");
    if (r.topk_group < 0 || r.topk_group > r.n_group)
      return fail(BH_HEX_ERR_VALUE, std::string(who) + ": topk_group must be in 0..n_group");
    if (r.sigmoid && r.n_group > 1 && k > (r.topk_group ? r.topk_group : r.n_group) * (E / r.n_group))
      return fail(BH_HEX_ERR_VALUE, std::string(who) + ": k exceeds the experts of the kept groups");
  }
  *out = r;
  return BH_HEX_OK;
}

template <int IDT>
static void select_ldt(int ldt, dim3 grid, hipStream_t st, const void* logits, int64_t s_lt, int64_t T, int32_t E,
                       int32_t k, const Routing& r, float* w, void* ids) {
  if (ldt == BH_HEX_F32)
    hipLaunchKernelGGL((route_select_kernel<BH_HEX_F32, IDT>), grid, dim3(256), 0, st, logits, s_lt, T, E, k, r, w, ids);
  else if (ldt == BH_HEX_BF16)
    hipLaunchKernelGGL((route_select_kernel<BH_HEX_BF16, IDT>), grid, dim3(256), 0, st, logits, s_lt, T, E, k, r, w, ids);
  else
    hipLaunchKernelGGL((route_select_kernel<BH_HEX_F16, IDT>), grid, dim3(256), 0, st, logits, s_lt, T, E, k, r, w, ids);
}

static int route_select(const char* who, const void* logits, int32_t logits_dtype, int64_t s_lt, int64_t T, int32_t E,
                        int32_t k, const Routing& r, float* topk_w, void* topk_ids, int32_t ids_dtype, void* stream) {
  if (T < 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": negative token count");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ids dtype must be I32 or I64");
  if (logits_dtype != BH_HEX_F32 && logits_dtype != BH_HEX_BF16 && logits_dtype != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": logits dtype must be F32, BF16 or F16");
  if (T == 0) return BH_HEX_OK;
  if (!logits || !topk_w || !topk_ids) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  if (s_lt < E) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": logits row stride below the expert count");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)cdiv(T, 4));
  if (ids_dtype == BH_HEX_I64) select_ldt<BH_HEX_I64>(logits_dtype, grid, st, logits, s_lt, T, E, k, r, topk_w, topk_ids);
  else select_ldt<BH_HEX_I32>(logits_dtype, grid, st, logits, s_lt, T, E, k, r, topk_w, topk_ids);
  return check_launch(who);
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_route_topk(const void* logits, int32_t logits_dtype, int64_t s_lt, int64_t T, int32_t E, int32_t k,
                                 int32_t renormalize, float* topk_w, void* topk_ids, int32_t ids_dtype, void* stream) {
  const bh_hex_routing soft{BH_HEX_SCORE_SOFTMAX, renormalize, 1, 0, 1.0f, nullptr};
  Routing r;
  if (int rc = check_routing("bh_hex_route_topk", E, k, &soft, &r)) return rc;
  return route_select("bh_hex_route_topk", logits, logits_dtype, s_lt, T, E, k, r, topk_w, topk_ids, ids_dtype, stream);
}

extern "C" int bh_hex_route_select(const void* logits, int32_t logits_dtype, int64_t s_lt, int64_t T, int32_t E,
                                   int32_t k, const bh_hex_routing* routing, float* topk_w, void* topk_ids,
                                   int32_t ids_dtype, void* stream) {
  Routing r;
  if (int rc = check_routing("bh_hex_route_select", E, k, routing, &r)) return rc;
  return route_select("bh_hex_route_select", logits, logits_dtype, s_lt, T, E, k, r, topk_w, topk_ids, ids_dtype, stream);
}

extern "C" int64_t bh_hex_route_gemm_workspace(int64_t T) { return T < 0 ? -1 : cdiv(T, 16) * 16; }

extern "C" int bh_hex_route_gemm(const void* x, int32_t x_dtype, int64_t s_xm, const void* w_router, int64_t s_we,
                                 int64_t T, int32_t H, int32_t E, int32_t k, const bh_hex_routing* routing,
                                 float* logits, int64_t s_lt, float* topk_w, void* topk_ids, int32_t ids_dtype,
                                 int32_t* counters, int64_t n_counters, void* stream) {
  const char* who = "bh_hex_route_gemm";
  Routing r;
  if (int rc = check_routing(who, E, k, routing, &r)) return rc;
  if (T < 0 || H <= 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes");
  if (x_dtype != BH_HEX_BF16 && x_dtype != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": x and the router weight must be BF16 or F16");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ids dtype must be I32 or I64");
  if (H % 32) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": the hidden size must be a multiple of 32");
  if (T == 0) return BH_HEX_OK;
  if (!x || !w_router || !logits || !topk_w || !topk_ids) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  if (s_xm < H || s_we < H || s_lt < E) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": row strides below the widths");
  if (s_xm % 8 || s_we % 8 || !aligned(x, 16) || !aligned(w_router, 16))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": x and router rows must be 16-byte aligned");
  if (T * s_xm * 2 > (int64_t)kMaxRecords || (int64_t)E * s_we * 2 > (int64_t)kMaxRecords ||
      T * s_lt * 4 > (int64_t)kMaxRecords || T > INT32_MAX / 2)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": tensors over 2 GiB");
  if (!counters || n_counters < cdiv(T, 16) * 16)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": counters smaller than bh_hex_route_gemm_workspace() asks");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)cdiv(T, 16), (unsigned)cdiv(E, 16));
  const uint16_t* xs = reinterpret_cast<const uint16_t*>(x);
  const uint16_t* ws = reinterpret_cast<const uint16_t*>(w_router);
#define BH_RG(ADT, IDT)                                                                                              \
  hipLaunchKernelGGL((route_gemm_kernel<ADT, IDT>), grid, dim3(256), 0, st, xs, s_xm, ws, s_we, (int32_t)T, H, E, k, r, \
                     logits, s_lt, topk_w, topk_ids, counters)
  if (x_dtype == BH_HEX_BF16) {
    if (ids_dtype == BH_HEX_I64) BH_RG(BH_HEX_BF16, BH_HEX_I64); else BH_RG(BH_HEX_BF16, BH_HEX_I32);
  } else {
    if (ids_dtype == BH_HEX_I64) BH_RG(BH_HEX_F16, BH_HEX_I64); else BH_RG(BH_HEX_F16, BH_HEX_I32);
  }
#undef BH_RG
  return check_launch(who);
}
