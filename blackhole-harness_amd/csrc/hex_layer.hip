// A whole decode-regime HEX MoE layer in one launch: slot plan, gate/up with SiLU, down with
// the top-k weight, and the k-slot sum.
//
// Replaces, for one tier and up to 512 slots, the sequence hex_moe_fused runs
// (runtime/blackhole_runtime/hex_moe.py:304-325): align (201-222), the two _hex_moe_kernel
// launches (322, 324) and y.view(T, k, H).sum(1) (325). Four launches become one; the down
// phase's weight loads start while the last gate/up items finish, and each token's sum runs as
// soon as its k slots are written.
//
//  * Plan. Every workgroup builds the same plan of 16-slot expert blocks in LDS: slots of
//    experts with a tier entry, grouped by expert (ascending) in slot order, each expert's run
//    padded to whole blocks. Uncovered slots get no block and add nothing to the sum.
//  * Work. The gate/up units and then the down units are cut into ranges exactly as the
//    per-projection kernels cut them (hex_range.h). Workgroups take ranges by ticket from one
//    counter, gate/up ranges first, so every gate/up range is held by a running workgroup
//    before any down range is handed out: the waits below always end, however many of the
//    grid's workgroups are resident.
//  * Hand-over. A gate/up range counts its finished items per plan block after its stores are
//    complete; a down range waits (bounded) for its blocks' counts to reach the block's row
//    tiles before it loads their activations. Activations and y rows cross workgroups through
//    device-coherent stores and loads.
//  * Sum. A down range counts its finished slots per (token, 256-row tile); the last arrival
//    adds the token's y rows in slot order in float32 and rounds once, as the sum kernel does.
//  * The last workgroup to leave clears the tickets and block counts; every other counter is
//    cleared by its last user. A bounded wait that gives up sets ctl[32] (sticky) and the
//    launch's output is then invalid.
#include <string>

#include "hex_range.h"

namespace bh {

constexpr int kLayerMaxSlots = 512;    // T * k
constexpr int kLayerMaxBlocks = 320;   // 16-slot blocks of the plan
constexpr int kLayerMt = 1;            // 16-slot blocks
constexpr int kCtl = 64;               // control words: [0] ticket, [16] workgroups out, [32] flag

struct LayerArgs {
  MoeArgs glu, down;     // gate/up: x -> act; down: act -> y (their plan pointers are unused)
  const void* ids;       // topk ids [T, k]
  int32_t ids_i64;
  int32_t T, k;
  int32_t* ctl;
  LayerPtrs lp;          // block counts [kLayerMaxBlocks], token counts [T, down row tiles],
                         // the flag ctl + 32, out [T, H]
};

template <int BITS>
struct LayerSmem {
  union Phase {
    MoeSmem<BITS, true, kLayerMt> glu;
    MoeSmem<BITS, false, kLayerMt> down;
  } ph;
  int sid[kLayerMaxBlocks * 16];   // slot rows of the plan's blocks, S for padding
  int eid[kLayerMaxBlocks];        // global expert of each block
  int lut[kMaxExperts];            // the tier lookup
  int cnt[kMaxExperts];            // covered slots per expert, then the expert's first block
  int key[kLayerMaxSlots];         // expert of each covered slot, -1 for none
  int tgt[kLayerMaxSlots];         // covered slots per token
  int done[kMaxDone];
  int comp[kMaxDone * 16];
  int used, n_comp, n_done, ticket, last;
};

// The plan, identical in every workgroup (no atomics decide an order).
template <int BITS>
__device__ __forceinline__ void layer_plan(const LayerArgs& la, LayerSmem<BITS>& sm) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int S = la.T * la.k, E = la.glu.n_experts;
  for (int e = tid; e < E; e += kThreads) {
    sm.lut[e] = la.glu.lookup[e];
    sm.cnt[e] = 0;
  }
  int64_t id = -1;
  if (tid < S)
    id = la.ids_i64 ? reinterpret_cast<const int64_t*>(la.ids)[tid] : reinterpret_cast<const int32_t*>(la.ids)[tid];
  __syncthreads();
  int key = -1;
  if (tid < S) {
    if (id >= 0 && id < E && sm.lut[id] >= 0) key = (int)id;
    sm.key[tid] = key;
  }
  __syncthreads();
  int rank = 0;                      // earlier slots of the same expert
  if (key >= 0) {
    atomicAdd(&sm.cnt[key], 1);
    for (int j = 0; j < tid; ++j) rank += sm.key[j] == key;
  }
  for (int t = tid; t < la.T; t += kThreads) {
    int c = 0;
    for (int j = 0; j < la.k; ++j) c += sm.key[t * la.k + j] >= 0;
    sm.tgt[t] = c;
  }
  __syncthreads();
  if (tid < kWave) {                 // block starts: lane l scans experts [16 l, 16 l + 16)
    constexpr int per = kMaxExperts / kWave;
    const int e0 = lane * per;
    int nb[per];
    int sum = 0;
#pragma unroll
    for (int q = 0; q < per; ++q) {
      nb[q] = e0 + q < E ? (sm.cnt[e0 + q] + 15) >> 4 : 0;
      sum += nb[q];
    }
    int incl = sum;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += o;
    }
    int start = incl - sum;
#pragma unroll
    for (int q = 0; q < per; ++q) {
      if (e0 + q < E) {
        sm.cnt[e0 + q] = start;
        for (int r = 0; r < nb[q]; ++r) sm.eid[start + r] = e0 + q;
        start += nb[q];
      }
    }
    if (lane == kWave - 1) sm.used = incl;
  }
  __syncthreads();
  for (int r = tid; r < sm.used * 16; r += kThreads) sm.sid[r] = S;
  __syncthreads();
  if (key >= 0) sm.sid[sm.cnt[key] * 16 + rank] = tid;
  // tokens without a covered slot sum nothing: their rows are zero (one workgroup each)
  const int H = la.down.N;
  for (int t = blockIdx.x; t < la.T; t += gridDim.x)
    if (sm.tgt[t] == 0)
      for (int c = tid * 4; c < H; c += kThreads * 4)
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(la.lp.out) + t * la.lp.s_ot + c) = u32x2{0u, 0u};
  __syncthreads();
}

template <int BITS, int ADT, int SB>
__global__ __launch_bounds__(kThreads) void hex_layer_kernel(LayerArgs la) {
  __shared__ LayerSmem<BITS> sm;
  const int tid = threadIdx.x;
  int first = 0;
  if (tid == 0) first = __hip_atomic_fetch_add(la.ctl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  layer_plan<BITS>(la, sm);
  if (tid == 0) sm.ticket = first;
  __syncthreads();

  int64_t t = sm.ticket;
  for (;;) {
    // The arguments are read through an index the compiler cannot see to be 0, so each range
    // loads its own phase's arguments instead of both phases' staying live across the loop
    // (they would not fit the scalar registers).
    int z, rtid;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    asm volatile("v_mov_b32 %0, %1" : "=v"(rtid) : "v"(tid));   // per-lane values: recomputed per range
    const LayerArgs& ar = (&la)[z];
    const int64_t used = sm.used;
    const Ranges rg = moe_ranges(used, ar.glu.N, ar.glu.K, gridDim.x);
    const Ranges rd = moe_ranges(used, ar.down.N, ar.down.K, gridDim.x);
    if (t >= rg.G + rd.G) break;
    int nxt = 0;                     // the next ticket is in flight during this range
    if (tid == 0) nxt = __hip_atomic_fetch_add(ar.ctl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    LayerCtx lc;
    lc.p = &ar.lp;
    lc.done = sm.done;
    lc.comp = sm.comp;
    lc.n_comp = &sm.n_comp;
    lc.n_done = &sm.n_done;
    lc.key = sm.key;
    lc.tgt = sm.tgt;
    if (t < rg.G)
      moe_range<BITS, ADT, true, kLayerMt, SB, true, true>(ar.glu, sm.ph.glu, t, rg, sm.lut, sm.sid, sm.eid, lc, rtid);
    else
      moe_range<BITS, ADT, false, kLayerMt, SB, true, true>(ar.down, sm.ph.down, t - rg.G, rd, sm.lut, sm.sid, sm.eid,
                                                            lc, rtid);
    __syncthreads();                 // the range's LDS is free
    if (tid == 0) sm.ticket = nxt;
    __syncthreads();
    t = sm.ticket;
  }

  // the last workgroup out clears the tickets and the block counts for the next launch
  if (tid == 0)
    sm.last = __hip_atomic_fetch_add(la.ctl + 16, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
  __syncthreads();
  if (sm.last) {
    for (int b = tid; b < kLayerMaxBlocks; b += kThreads)
      __hip_atomic_store(la.lp.ready + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
      __hip_atomic_store(la.ctl, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(la.ctl + 16, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ----------------------------------------------------------------------------------- host side

// Workspace of the layer kernel: counters (control words, block counts, token counts, split
// items of both phases) and partial sums of both phases.
struct LayerWorkspace {
  int64_t ready, tokcnt, glu_cnt, down_cnt, counters;   // int32 offsets and total
  int64_t glu_part, partials;                           // float offset of the down partials, total
};

static int64_t layer_max_blocks(int64_t S, int64_t E) { return S / 16 + (E < S ? E : S); }

static LayerWorkspace layer_workspace(int64_t T, int64_t k, int64_t H, int64_t I, int64_t E) {
  const int64_t mb = layer_max_blocks(T * k, E);
  const int64_t g = device_cus();
  LayerWorkspace w;
  w.ready = kCtl;
  w.tokcnt = w.ready + kLayerMaxBlocks;
  w.glu_cnt = w.tokcnt + T * cdiv(H, kRows);
  w.down_cnt = w.glu_cnt + mb * cdiv(I, kRows) * kWaves;
  w.counters = w.down_cnt + mb * cdiv(H, kRows) * kWaves;
  w.glu_part = g * 2 * kWaves * part_floats<kLayerMt, 2>();
  w.partials = w.glu_part + g * 2 * kWaves * part_floats<kLayerMt, 1>();
  return w;
}

// Longest range of either phase, in items and blocks, at the plan's largest size.
static bool layer_ranges_fit(int64_t mb, int64_t N, int64_t K, int64_t grid) {
  const Ranges r = moe_ranges(mb, (int)N, (int)K, grid);
  const int64_t nrt = cdiv(N, kRows), nun = cdiv(K / kHexBlock, 8);
  const int64_t units = cdiv(r.U, r.G);
  return cdiv(units, nun) + 1 <= kMaxDone && cdiv(units, nrt * nun) + 2 <= kMaxBlk16 / kLayerMt;
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_moe_layer_workspace(int64_t T, int32_t k, int64_t H, int64_t I, int32_t n_experts,
                                          int64_t* n_counters, int64_t* n_partials) {
  if (T < 0 || k <= 0 || H <= 0 || I <= 0 || n_experts <= 0 || !n_counters || !n_partials)
    return fail(BH_HEX_ERR_VALUE, "bh_hex_moe_layer_workspace: bad arguments");
  const LayerWorkspace w = layer_workspace(T, k, H, I, n_experts);
  *n_counters = w.counters;
  *n_partials = w.partials;
  return BH_HEX_OK;
}

extern "C" int bh_hex_moe_layer(const void* x, int32_t x_dtype, int64_t s_xm, const void* topk_ids, int32_t ids_dtype,
                                const float* topk_w, int64_t T, int32_t k, const bh_hex_proj* gate,
                                const bh_hex_proj* up, const bh_hex_proj* down, int32_t bits, int64_t H, int64_t I,
                                const int32_t* lookup, int32_t n_experts, void* act, int64_t s_am, float* y,
                                int64_t s_ym, void* out, int64_t s_ot, int32_t* counters, int64_t n_counters,
                                float* partials, int64_t n_partials, void* stream) {
  const char* who = "bh_hex_moe_layer";
  if (bits != 3 && bits != 4) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": bits must be 3 or 4");
  if (x_dtype != BH_HEX_BF16 && x_dtype != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": activations must be BF16 or F16");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ids dtype must be I32 or I64");
  if (T < 0 || k <= 0 || H <= 0 || I <= 0 || H > (1 << 30) || I > (1 << 30) || n_experts <= 0)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes");
  if (n_experts > kMaxExperts) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": at most 1024 experts");
  const int64_t S = T * k;
  const int64_t mb = layer_max_blocks(S, n_experts);
  if (S > kLayerMaxSlots || mb > kLayerMaxBlocks)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": more slots than one launch plans (512)");
  int sb = 0, words = 1;
  if (int rc = proj_setup(who, gate, bits, H, &sb, &words)) return rc;
  if (int rc = proj_setup(who, up, bits, H, &sb, &words)) return rc;
  const int sb_glu = sb;
  sb = 0;
  if (int rc = proj_setup(who, down, bits, I, &sb, &words)) return rc;
  if (sb != sb_glu) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": projections with different scale blocks");
  if ((H / kHexBlock) % 8 || (I / kHexBlock) % 8 || !words)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": widths must be multiples of 256 with aligned scale rows");
  if (!x || !topk_ids || !topk_w || !lookup || !act || !y || !out)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  if (s_xm % 8 || !aligned(x, 16) || s_am % 8 || !aligned(act, 16) || s_ym % 4 || !aligned(y, 16) || s_ot % 4 ||
      !aligned(out, 8))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": x, act and y rows must be 16-byte aligned, out rows 8-byte");
  if (T * s_xm * 2 > 0x7FFFFFFF || S * s_am * 2 > 0x7FFFFFFF || S * s_ym * 4 > 0x7FFFFFFF)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": x, act or y over 2 GiB");
  const int64_t grid = device_cus();
  if (!layer_ranges_fit(mb, I, H, grid) || !layer_ranges_fit(mb, H, I, grid))
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ranges too long for this device");
  const LayerWorkspace w = layer_workspace(T, k, H, I, n_experts);
  if (!counters || !partials || n_counters < w.counters || n_partials < w.partials)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": workspace smaller than bh_hex_moe_layer_workspace() asks");
  if (!aligned(partials, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": partials must be 16-byte aligned");
  if (w.partials * 4 > 0x7FFFFFFF) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": workspace too large");
  if (T == 0) return BH_HEX_OK;

  LayerArgs la{};
  MoeArgs& g = la.glu;
  g.x = reinterpret_cast<const uint16_t*>(x);
  g.s_xm = s_xm;
  g.out = act;
  g.s_om = s_am;
  g.w0 = *gate;
  g.w1 = *up;
  g.lookup = lookup;
  g.num_slots = S;
  g.n_experts = n_experts;
  g.a_div = k;
  g.N = (int32_t)I;
  g.K = (int32_t)H;
  g.scale_words = words;
  g.part = partials;
  g.counters = counters + w.glu_cnt;
  MoeArgs& d = la.down;
  d.x = reinterpret_cast<const uint16_t*>(act);
  d.s_xm = s_am;
  d.out = y;
  d.s_om = s_ym;
  d.w0 = *down;
  d.w1 = *down;
  d.lookup = lookup;
  d.topk_w = topk_w;
  d.num_slots = S;
  d.n_experts = n_experts;
  d.a_div = 1;
  d.N = (int32_t)H;
  d.K = (int32_t)I;
  d.scale_words = words;
  d.part = partials + w.glu_part;
  d.counters = counters + w.down_cnt;
  la.ids = topk_ids;
  la.ids_i64 = ids_dtype == BH_HEX_I64;
  la.T = (int32_t)T;
  la.k = k;
  la.ctl = counters;
  la.lp.ready = counters + w.ready;
  la.lp.tokcnt = counters + w.tokcnt;
  la.lp.flag = counters + 32;
  la.lp.out = out;
  la.lp.s_ot = s_ot;
  la.lp.k = k;
  la.lp.glu_tiles = (int32_t)cdiv(I, kRows);

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 gd((unsigned)grid), bd(kThreads);
#define BH_LAYER(B, A, SBV) hipLaunchKernelGGL((hex_layer_kernel<B, A, SBV>), gd, bd, 0, st, la)
  if (bits == 4) {
    if (x_dtype == BH_HEX_BF16) {
      if (sb == 1) BH_LAYER(4, BH_HEX_BF16, 1); else BH_LAYER(4, BH_HEX_BF16, 4);
    } else {
      if (sb == 1) BH_LAYER(4, BH_HEX_F16, 1); else BH_LAYER(4, BH_HEX_F16, 4);
    }
  } else {
    if (x_dtype == BH_HEX_BF16) {
      if (sb == 1) BH_LAYER(3, BH_HEX_BF16, 1); else BH_LAYER(3, BH_HEX_BF16, 4);
    } else {
      if (sb == 1) BH_LAYER(3, BH_HEX_F16, 1); else BH_LAYER(3, BH_HEX_F16, 4);
    }
  }
#undef BH_LAYER
  return check_launch(who);
}
