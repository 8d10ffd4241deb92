// Fused HEX expert GEMMs on the CDNA4 matrix cores (one launch per projection), and the k-slot
// reduction.
//
// Replaces the reference's _hex_moe_kernel (runtime/blackhole_runtime/hex_moe.py:109-151) in
// both roles (GLU gate/up with SiLU, and down with the top-k weight) and the torch sum at
// hex_moe.py:325. The decode-regime kernel is one persistent launch over the ranges of
// hex_range.h, one range per workgroup; the 128-slot prefill kernels are in hex_gemm.hip.
#include <algorithm>
#include <mutex>
#include <string>

#include "hex_range.h"

namespace bh {

template <int BITS, int ADT, bool GLU, int MT, int SB, bool KF>
__global__ __launch_bounds__(kThreads) void hex_moe_kernel(MoeArgs a) {
  __shared__ MoeSmem<BITS, GLU, MT> sm;
  touch_args<MoeArgs>();
  moe_range<BITS, ADT, GLU, MT, SB, KF>(a, sm, blockIdx.x, threadIdx.x);
}

// ----------------------------------------------------------------------------------- reduction

// Four y values of a slot row as float32 (YDT: F32, BF16 or F16).
template <int YDT>
__device__ __forceinline__ f32x4 y4(const void* y, int64_t at) {
  if constexpr (YDT == BH_HEX_F32) {
    return *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(y) + at);
  } else {
    const u32x2 v = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(y) + at);
    return f32x4{from_bits<YDT>(v[0] & 0xFFFFu), from_bits<YDT>(v[0] >> 16), from_bits<YDT>(v[1] & 0xFFFFu),
                 from_bits<YDT>(v[1] >> 16)};
  }
}

// Eight 16-bit y values of a slot row (one 16-byte load) as two float32 quads.
template <int YDT>
__device__ __forceinline__ void y8(const void* y, int64_t at, f32x4& lo, f32x4& hi) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(y) + at);
  lo = f32x4{from_bits<YDT>(v[0] & 0xFFFFu), from_bits<YDT>(v[0] >> 16), from_bits<YDT>(v[1] & 0xFFFFu),
             from_bits<YDT>(v[1] >> 16)};
  hi = f32x4{from_bits<YDT>(v[2] & 0xFFFFu), from_bits<YDT>(v[2] >> 16), from_bits<YDT>(v[3] & 0xFFFFu),
             from_bits<YDT>(v[3] >> 16)};
}

// 16-bit y in rows of multiples of 8 values: eight outputs per thread, each slot row read with
// one 16-byte load (the four-output kernel below reads 8 bytes per load). The same sums in the
// same order.
template <int ODT, int IDT, int YDT>
__global__ __launch_bounds__(256) void moe_reduce8_kernel(const void* __restrict__ y, int64_t s_ym,
                                                          const void* __restrict__ ids, int32_t n_experts, int32_t k,
                                                          int64_t H, void* __restrict__ out, int64_t s_ot) {
  const int64_t t = blockIdx.y;
  const int64_t h = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (h >= H) return;
  f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < k; j0 += 8) {
    int64_t id[8];
    f32x4 v0[8], v1[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int64_t s = t * k + j0 + d;
      if (j0 + d < k) {
        if constexpr (IDT == BH_HEX_I64) id[d] = reinterpret_cast<const int64_t*>(ids)[s];
        else id[d] = reinterpret_cast<const int32_t*>(ids)[s];
        y8<YDT>(y, s * s_ym + h, v0[d], v1[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < 8; ++d)
      if (j0 + d < k && id[d] >= 0 && id[d] < n_experts) {
        a0 += v0[d];
        a1 += v1[d];
      }
  }
  if constexpr (ODT == BH_HEX_F32) {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + t * s_ot + h) = a0;
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + t * s_ot + h + 4) = a1;
  } else {
    u32x4 v;
    v[0] = to_bits<ODT>(a0[0]) | (to_bits<ODT>(a0[1]) << 16);
    v[1] = to_bits<ODT>(a0[2]) | (to_bits<ODT>(a0[3]) << 16);
    v[2] = to_bits<ODT>(a1[0]) | (to_bits<ODT>(a1[1]) << 16);
    v[3] = to_bits<ODT>(a1[2]) | (to_bits<ODT>(a1[3]) << 16);
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(out) + t * s_ot + h) = v;
  }
}

template <int ODT, int IDT, int YDT>
__global__ __launch_bounds__(256) void moe_reduce_kernel(const void* __restrict__ y, int64_t s_ym,
                                                         const void* __restrict__ ids, int32_t n_experts, int32_t k,
                                                         int64_t H, void* __restrict__ out, int64_t s_ot) {
  const int64_t t = blockIdx.y;
  const int64_t h = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (h >= H) return;
  // Eight slots at a time, their ids and y rows loaded together (a y row of a slot with an
  // invalid id is in bounds but unwritten: it is read and dropped); added in slot order.
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < k; j0 += 8) {
    int64_t id[8];
    f32x4 v[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int64_t s = t * k + j0 + d;
      if (j0 + d < k) {
        if constexpr (IDT == BH_HEX_I64) id[d] = reinterpret_cast<const int64_t*>(ids)[s];
        else id[d] = reinterpret_cast<const int32_t*>(ids)[s];
        v[d] = y4<YDT>(y, s * s_ym + h);
      }
    }
#pragma unroll
    for (int d = 0; d < 8; ++d)
      if (j0 + d < k && id[d] >= 0 && id[d] < n_experts) acc += v[d];
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
  // whole 256-input units with aligned scale rows: no tail checks, one load per unit's scales
  const bool kf = (a.K / kHexBlock) % 8 == 0 && a.scale_words;
  const dim3 block(kThreads);
  if (sb == 1) {
    if (kf) hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 1, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 1, false>), grid, block, 0, st, a);
  } else {
    if (kf) hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 4, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((hex_moe_kernel<BITS, ADT, GLU, MT, 4, false>), grid, block, 0, st, a);
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

int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Persistent grid: one workgroup per compute unit, fewer when the plan's units (an upper bound
// from num_blocks) would give a workgroup fewer than kMinUnits units, and enough that no
// workgroup's range spans more expert blocks than it stages in LDS (64 / MT).
static int64_t moe_grid(int64_t num_blocks, int64_t n_out, int64_t n_in, int mt) {
  const int64_t units = num_blocks * cdiv(n_out, kRows) * cdiv(cdiv(n_in, kHexBlock), 8);
  int64_t g = cdiv(units, kMinUnits);
  if (g > device_cus()) g = device_cus();
  const int64_t min_g = cdiv(num_blocks, kMaxBlk16 / mt - 2);
  if (g < min_g) g = min_g;
  return g > 0 ? g : 1;
}

// Workspace of one launch: arrival counters (one per item, 64 bytes apart) and partial-sum tiles
// (two per workgroup and wave), as two separate buffers so calls of any shape can share them.
struct Workspace {
  int64_t counters, partials;      // int32 counters, float partials
};

static Workspace workspace_layout(int64_t num_blocks, int64_t n_out, int64_t n_in, int mt, bool glu) {
  Workspace w;
  w.counters = num_blocks * cdiv(n_out, kRows) * kWaves;
  w.partials = moe_grid(num_blocks, n_out, n_in, mt) * 2 * kWaves * (int64_t)mt * (glu ? 2 : 1) * kWave * 4;
  return w;
}

// Where a launch's slot plan comes from: the align kernel's outputs (sid, eid, npp over
// num_blocks blocks), or the routing ids themselves (ids), which the decode kernels sort in
// their own workgroups.
struct PlanSrc {
  const int32_t* sid;
  const int32_t* eid;
  int64_t num_blocks;
  const int32_t* npp;
  const void* ids;
  int32_t ids_dtype;
};

// Shared argument checks of the fused entry points; fills the plan part of MoeArgs. With ids the
// plan's block count is align()'s upper bound ceil(S / block_m) + min(n_experts, S).
static int check_moe(const char* who, int32_t bits, int32_t adt, int64_t n_out, int64_t n_in, PlanSrc& pl,
                     const int32_t* lookup, int32_t n_experts, int64_t num_slots, const bh_hex_tile* tile, int* mt,
                     MoeArgs& a) {
  if (bits != 3 && bits != 4) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": bits must be 3 or 4");
  if (adt != BH_HEX_BF16 && adt != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": activations must be BF16 or F16");
  if (!tile) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null tile");
  if (tile->block_m != 16 && tile->block_m != 32 && tile->block_m != 64 && tile->block_m != 128)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m must be 16, 32, 64 or 128");
  if (tile->block_n != kRows || tile->k_split != 1)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_n must be 256 and k_split 1");
  if (n_out <= 0 || n_out > (1 << 30) || n_in > (1 << 30)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad width");
  if (n_experts <= 0 || num_slots < 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad plan sizes");
  if (n_experts > kMaxExperts)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": at most 1024 experts");
  if (pl.ids) {
    if (tile->block_m == 128)
      return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m 128 takes a plan from the align kernel");
    if (num_slots > kPlanMaxSlots)
      return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": the kernels sort at most 1024 slots themselves");
    if (pl.ids_dtype != BH_HEX_I32 && pl.ids_dtype != BH_HEX_I64)
      return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ids dtype must be I32 or I64");
    if (!lookup) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null lookup");
    pl.num_blocks = cdiv(num_slots, tile->block_m) + std::min<int64_t>(n_experts, num_slots);
  } else {
    if (pl.num_blocks < 0 || pl.num_blocks > INT32_MAX) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad plan sizes");
    if (pl.num_blocks > 0 && (!pl.sid || !pl.eid || !pl.npp || !lookup))
      return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null plan pointer");
  }
  *mt = tile->block_m / 16;
  a.sid = pl.sid;
  a.eid = pl.eid;
  a.npp = pl.npp;
  a.ids = pl.ids;
  a.ids_i64 = pl.ids_dtype == BH_HEX_I64;
  a.lookup = lookup;
  a.n_experts = n_experts;
  a.num_slots = num_slots;
  a.N = (int32_t)n_out;
  a.K = (int32_t)n_in;
  return BH_HEX_OK;
}

// Points the kernel at the caller's workspace.
static int attach_workspace(const char* who, int32_t* counters, int64_t n_counters, float* partials,
                            int64_t n_partials, int64_t num_blocks, int64_t n_out, int64_t n_in, int mt, bool glu,
                            MoeArgs& a, dim3* grid) {
  const Workspace w = workspace_layout(num_blocks, n_out, n_in, mt, glu);
  if (!counters || !partials || n_counters < w.counters || n_partials < w.partials)
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": workspace smaller than bh_hex_moe_workspace() asks");
  if (!aligned(partials, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": partials must be 16-byte aligned");
  if (w.partials * 4 > (int64_t)kMaxRecords) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": plan too large");
  // the kernels cut the units into ranges in 32-bit arithmetic: units x workgroups must fit in 31 bits
  const int64_t g = moe_grid(num_blocks, n_out, n_in, mt);
  const int64_t units = num_blocks * cdiv(n_out, kRows) * cdiv(cdiv(n_in, kHexBlock), 8);
  if (units * (g + 1) >= (int64_t)1 << 31)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": plan too large for the decode kernels");
  a.counters = counters;
  a.part = partials;
  *grid = dim3((unsigned)g);
  return BH_HEX_OK;
}

int proj_setup(const char* who, const bh_hex_proj* w, int bits, int64_t n_out, int64_t n_in, int* sb, int* words) {
  int block = 0;
  if (int rc = check_proj(w, n_in, who, &block)) return rc;
  if (block != 32 && block != 128)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": fused kernels take scale blocks of 32 or 128 inputs");
  if (*sb && *sb != block / 32) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": gate and up scale blocks differ");
  *sb = block / 32;
  // one expert's matrix is one buffer resource of at most kMaxRecords bytes
  if (n_out * w->s_in * 4 > (int64_t)kMaxRecords || n_out * w->s_bn > (int64_t)kMaxRecords)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": expert matrix over 2 GiB");
  if (bits == 4 && (w->s_ie % 4 || w->s_in % 4 || !aligned(w->idx, 16)))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": 4-bit idx rows must be 16-byte aligned");
  // a unit's scales in one load: 8 bytes at 32-input blocks, 2 bytes at 128-input blocks
  const int sw = block == 32 ? 8 : 2;
  if (w->s_bn % sw || w->s_be % sw || !aligned(w->block_scale, sw)) *words = 0;
  return BH_HEX_OK;
}


static int moe_glu(const char* who, const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                   const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out, int64_t n_in, PlanSrc pl,
                   const int32_t* lookup, int32_t n_experts, int64_t num_slots, int32_t a_div, const bh_hex_tile* tile,
                   int32_t* counters, int64_t n_counters, float* partials, int64_t n_partials, void* stream) {
  MoeArgs a{};
  int mt = 0, sb = 0, words = 1;
  int rc = check_moe(who, bits, x_dtype, n_out, n_in, pl, lookup, n_experts, num_slots, tile, &mt, a);
  if (rc) return rc;
  if ((rc = proj_setup(who, gate, bits, n_out, n_in, &sb, &words))) return rc;
  if ((rc = proj_setup(who, up, bits, n_out, n_in, &sb, &words))) return rc;
  if (a_div <= 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": a_div must be positive");
  if (!x || !act) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null activation pointer");
  if (s_xm % 8 || !aligned(x, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": x rows must be 16-byte aligned");
  if (cdiv(num_slots, a_div) * s_xm * 2 > (int64_t)kMaxRecords)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": x over 2 GiB");
  if (pl.num_blocks == 0 || num_slots == 0) return BH_HEX_OK;
  a.x = reinterpret_cast<const uint16_t*>(x);
  a.s_xm = s_xm;
  a.out = act;
  a.s_om = s_am;
  a.w0 = *gate;
  a.w1 = *up;
  a.a_div = a_div;
  a.scale_words = words;
  if (mt == kGemmMt) return gemm_run(who, true, bits, x_dtype, sb, a, pl.num_blocks, reinterpret_cast<hipStream_t>(stream));
  dim3 grid;
  if ((rc = attach_workspace(who, counters, n_counters, partials, n_partials, pl.num_blocks, n_out, n_in, mt, true, a,
                             &grid))) return rc;
  launch_moe<true>(bits, x_dtype, mt, sb, grid, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(who);
}

static int moe_down(const char* who, const void* act, int32_t act_dtype, int64_t s_am, void* y, int32_t y_dtype,
                    int64_t s_ym, const bh_hex_proj* down, int32_t bits, int64_t n_out, int64_t n_in, PlanSrc pl,
                    const int32_t* lookup, int32_t n_experts, int64_t num_slots, const float* topk_w,
                    const bh_hex_tile* tile, int32_t* counters, int64_t n_counters, float* partials, int64_t n_partials,
                    void* stream) {
  MoeArgs a{};
  int mt = 0, sb = 0, words = 1;
  int rc = check_moe(who, bits, act_dtype, n_out, n_in, pl, lookup, n_experts, num_slots, tile, &mt, a);
  if (rc) return rc;
  if ((rc = proj_setup(who, down, bits, n_out, n_in, &sb, &words))) return rc;
  if (!act || !y || !topk_w) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null pointer");
  if (y_dtype != BH_HEX_F32 && y_dtype != act_dtype)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": y dtype must be F32 or the activation dtype");
  if (s_am % 8 || !aligned(act, 16)) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": act rows must be 16-byte aligned");
  if (num_slots * s_am * 2 > (int64_t)kMaxRecords)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": act over 2 GiB");
  if (pl.num_blocks == 0 || num_slots == 0) return BH_HEX_OK;
  a.x = reinterpret_cast<const uint16_t*>(act);
  a.s_xm = s_am;
  a.out = y;
  a.s_om = s_ym;
  a.y16 = y_dtype != BH_HEX_F32;
  a.w0 = *down;
  a.w1 = *down;
  a.topk_w = topk_w;
  a.a_div = 1;
  a.scale_words = words;
  if (mt == kGemmMt) return gemm_run(who, false, bits, act_dtype, sb, a, pl.num_blocks, reinterpret_cast<hipStream_t>(stream));
  dim3 grid;
  if ((rc = attach_workspace(who, counters, n_counters, partials, n_partials, pl.num_blocks, n_out, n_in, mt, false, a,
                             &grid))) return rc;
  launch_moe<false>(bits, act_dtype, mt, sb, grid, reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(who);
}

// ----------------------------------------------------------------------------------- static scratch

// The workspace of bh_hex_moe_glu_ids_noalloc: a static device array, one copy per device,
// held until the process ends. The first kScratchCounters words are the arrival counters
// (zero at load, zeroed again when a device is set up, and left zero by every call); the rest
// are partial sums (no initial value). 1 MiB of counters and 16 MiB of partials: the partials of
// a 16-slot gate/up launch on 256 workgroups (256 x 2 x 16 waves x 2 matrices x 64 lanes x 4).
constexpr int64_t kScratchCounters = 1 << 18;
constexpr int64_t kScratchPartials = 1 << 22;
static __device__ __align__(256) uint32_t scratch[kScratchCounters + kScratchPartials];

__global__ void zero_words_kernel(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static uint32_t* g_scratch[kMaxScratchDevices];   // device address of `scratch` per device

// The device address of the stream's device's scratch. Set up once per device, with that
// device current: the symbol's address is looked up (the array's name is only a host-side
// stand-in) and its counters are cleared by a fill kernel on `st`, ahead of the call's kernels.
static int scratch_for(const char* who, hipStream_t st, uint32_t** out) {
  int dev = 0;
  if (hipStreamGetDevice(st, &dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail(BH_HEX_ERR_HIP, std::string(who) + ": cannot tell the stream's device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return fail(BH_HEX_ERR_HIP, std::string(who) + ": hipGetDevice failed");
    if (cur != dev && hipSetDevice(dev) != hipSuccess)
      return fail(BH_HEX_ERR_HIP, std::string(who) + ": hipSetDevice failed");
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p) {
      hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(kScratchCounters, 256)), dim3(256), 0, st,
                         static_cast<uint32_t*>(p), kScratchCounters);
    }
    const hipError_t le = hipGetLastError();
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return fail(BH_HEX_ERR_HIP, std::string(who) + ": hipGetSymbolAddress(scratch): " + hipGetErrorString(e));
    if (le != hipSuccess) return fail(BH_HEX_ERR_HIP, std::string(who) + ": clearing the scratch: " + hipGetErrorString(le));
    g_scratch[dev] = static_cast<uint32_t*>(p);
  }
  *out = g_scratch[dev];
  return BH_HEX_OK;
}

}  // namespace bh

using namespace bh;

extern "C" int bh_hex_moe_glu(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                              const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out, int64_t n_in,
                              const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks,
                              const int32_t* npp, const int32_t* lookup, int32_t n_experts, int64_t num_slots,
                              int32_t a_div, const bh_hex_tile* tile, int32_t* counters, int64_t n_counters,
                              float* partials, int64_t n_partials, void* stream) {
  return moe_glu("bh_hex_moe_glu", x, x_dtype, s_xm, act, s_am, gate, up, bits, n_out, n_in,
                 PlanSrc{sorted_ids, expert_ids, num_blocks, npp, nullptr, 0}, lookup, n_experts, num_slots, a_div, tile,
                 counters, n_counters, partials, n_partials, stream);
}

extern "C" int bh_hex_moe_glu_ids(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                                  const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits, int64_t n_out,
                                  int64_t n_in, const void* topk_ids, int32_t ids_dtype, const int32_t* lookup,
                                  int32_t n_experts, int64_t num_slots, int32_t a_div, const bh_hex_tile* tile,
                                  int32_t* counters, int64_t n_counters, float* partials, int64_t n_partials,
                                  void* stream) {
  if (!topk_ids && num_slots > 0) return fail(BH_HEX_ERR_VALUE, "bh_hex_moe_glu_ids: null ids");
  return moe_glu("bh_hex_moe_glu_ids", x, x_dtype, s_xm, act, s_am, gate, up, bits, n_out, n_in,
                 PlanSrc{nullptr, nullptr, 0, nullptr, topk_ids ? topk_ids : x, ids_dtype}, lookup, n_experts,
                 num_slots, a_div, tile, counters, n_counters, partials, n_partials, stream);
}

extern "C" int bh_hex_moe_glu_ids_noalloc(const void* x, int32_t x_dtype, int64_t s_xm, void* act, int64_t s_am,
                                          const bh_hex_proj* gate, const bh_hex_proj* up, int32_t bits,
                                          int64_t n_out, int64_t n_in, const void* topk_ids, int32_t ids_dtype,
                                          const int32_t* lookup, int32_t n_experts, int64_t num_slots, int32_t a_div,
                                          const bh_hex_tile* tile, void* stream) {
  const char* who = "bh_hex_moe_glu_ids_noalloc";
  if (!topk_ids && num_slots > 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null ids");
  if (!tile) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": null tile");
  if (tile->block_m != 16 && tile->block_m != 32 && tile->block_m != 64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": block_m must be 16, 32 or 64");
  if (num_slots < 0 || num_slots > kPlanMaxSlots || n_experts <= 0 || n_experts > kMaxExperts || n_out <= 0 ||
      n_out > (1 << 30) || n_in <= 0 || n_in > (1 << 30))
    return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes (at most 1024 slots and 1024 experts)");
  const int64_t nb = cdiv(num_slots, tile->block_m) + std::min<int64_t>(n_experts, num_slots);
  const Workspace w = workspace_layout(nb, n_out, n_in, tile->block_m / 16, true);
  if (w.counters > kScratchCounters || w.partials > kScratchPartials)
    return fail(BH_HEX_ERR_UNSUPPORTED,
                std::string(who) + ": the launch needs " + std::to_string(w.counters) + " counters and " +
                    std::to_string(w.partials) + " partial sums; the static scratch holds " +
                    std::to_string(kScratchCounters) + " and " + std::to_string(kScratchPartials) +
                    " (use bh_hex_moe_glu_ids with a workspace)");
  uint32_t* s = nullptr;
  if (int rc = scratch_for(who, reinterpret_cast<hipStream_t>(stream), &s)) return rc;
  return moe_glu(who, x, x_dtype, s_xm, act, s_am, gate, up, bits, n_out, n_in,
                 PlanSrc{nullptr, nullptr, 0, nullptr, topk_ids ? topk_ids : x, ids_dtype}, lookup, n_experts,
                 num_slots, a_div, tile, reinterpret_cast<int32_t*>(s), kScratchCounters,
                 reinterpret_cast<float*>(s + kScratchCounters), kScratchPartials, stream);
}

extern "C" int bh_hex_moe_down(const void* act, int32_t act_dtype, int64_t s_am, void* y, int32_t y_dtype, int64_t s_ym,
                               const bh_hex_proj* down, int32_t bits, int64_t n_out, int64_t n_in,
                               const int32_t* sorted_ids, const int32_t* expert_ids, int64_t num_blocks,
                               const int32_t* npp, const int32_t* lookup, int32_t n_experts, int64_t num_slots,
                               const float* topk_w, const bh_hex_tile* tile, int32_t* counters, int64_t n_counters,
                               float* partials, int64_t n_partials, void* stream) {
  return moe_down("bh_hex_moe_down", act, act_dtype, s_am, y, y_dtype, s_ym, down, bits, n_out, n_in,
                  PlanSrc{sorted_ids, expert_ids, num_blocks, npp, nullptr, 0}, lookup, n_experts, num_slots, topk_w,
                  tile, counters, n_counters, partials, n_partials, stream);
}

extern "C" int bh_hex_moe_down_ids(const void* act, int32_t act_dtype, int64_t s_am, void* y, int32_t y_dtype,
                                   int64_t s_ym, const bh_hex_proj* down, int32_t bits, int64_t n_out, int64_t n_in,
                                   const void* topk_ids, int32_t ids_dtype, const int32_t* lookup, int32_t n_experts,
                                   int64_t num_slots, const float* topk_w, const bh_hex_tile* tile, int32_t* counters,
                                   int64_t n_counters, float* partials, int64_t n_partials, void* stream) {
  if (!topk_ids && num_slots > 0) return fail(BH_HEX_ERR_VALUE, "bh_hex_moe_down_ids: null ids");
  return moe_down("bh_hex_moe_down_ids", act, act_dtype, s_am, y, y_dtype, s_ym, down, bits, n_out, n_in,
                  PlanSrc{nullptr, nullptr, 0, nullptr, topk_ids ? topk_ids : act, ids_dtype}, lookup, n_experts,
                  num_slots, topk_w, tile, counters, n_counters, partials, n_partials, stream);
}

extern "C" int bh_hex_moe_workspace(int64_t num_blocks, int64_t n_out, int64_t n_in, int32_t block_m, int32_t glu,
                                    int64_t* n_counters, int64_t* n_partials) {
  if (num_blocks < 0 || n_out <= 0 || n_in <= 0 || !n_counters || !n_partials)
    return fail(BH_HEX_ERR_VALUE, "bh_hex_moe_workspace: bad arguments");
  if (block_m != 16 && block_m != 32 && block_m != 64 && block_m != 128)
    return fail(BH_HEX_ERR_UNSUPPORTED, "bh_hex_moe_workspace: block_m must be 16, 32, 64 or 128");
  if (block_m / 16 == kGemmMt) {     // the 128-slot kernels need no workspace
    *n_counters = 0;
    *n_partials = 0;
    return BH_HEX_OK;
  }
  const Workspace w = workspace_layout(num_blocks, n_out, n_in, block_m / 16, glu != 0);
  *n_counters = w.counters;
  *n_partials = w.partials;
  return BH_HEX_OK;
}

template <int ODT, int IDT>
static void reduce_ydt(int ydt, dim3 grid, hipStream_t st, const void* y, int64_t s_ym, const void* ids,
                       int32_t n_experts, int32_t k, int64_t H, void* out, int64_t s_ot) {
  // 16-bit y in 16-byte aligned rows of multiples of 8 values: the eight-output kernel
  const bool wide = ydt != BH_HEX_F32 && H % 8 == 0 && s_ym % 8 == 0 && s_ot % 8 == 0 && aligned(y, 16) &&
                    aligned(out, 16);
  if (wide) {
    const dim3 g8((unsigned)cdiv(H, 2048), grid.y);
    if (ydt == BH_HEX_BF16)
      hipLaunchKernelGGL((moe_reduce8_kernel<ODT, IDT, BH_HEX_BF16>), g8, dim3(256), 0, st, y, s_ym, ids, n_experts, k,
                         H, out, s_ot);
    else
      hipLaunchKernelGGL((moe_reduce8_kernel<ODT, IDT, BH_HEX_F16>), g8, dim3(256), 0, st, y, s_ym, ids, n_experts, k,
                         H, out, s_ot);
    return;
  }
  if (ydt == BH_HEX_F32)
    hipLaunchKernelGGL((moe_reduce_kernel<ODT, IDT, BH_HEX_F32>), grid, dim3(256), 0, st, y, s_ym, ids, n_experts, k, H,
                       out, s_ot);
  else if (ydt == BH_HEX_BF16)
    hipLaunchKernelGGL((moe_reduce_kernel<ODT, IDT, BH_HEX_BF16>), grid, dim3(256), 0, st, y, s_ym, ids, n_experts, k,
                       H, out, s_ot);
  else
    hipLaunchKernelGGL((moe_reduce_kernel<ODT, IDT, BH_HEX_F16>), grid, dim3(256), 0, st, y, s_ym, ids, n_experts, k, H,
                       out, s_ot);
}

extern "C" int bh_hex_moe_reduce(const void* y, int32_t y_dtype, int64_t s_ym, const void* topk_ids, int32_t ids_dtype,
                                 int32_t n_experts, int64_t T, int32_t k, int64_t H, void* out, int32_t out_dtype,
                                 int64_t s_ot, void* stream) {
  const char* who = "bh_hex_moe_reduce";
  if (T < 0 || k <= 0 || H <= 0) return fail(BH_HEX_ERR_VALUE, std::string(who) + ": bad sizes");
  if (y_dtype != BH_HEX_F32 && y_dtype != BH_HEX_BF16 && y_dtype != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": y dtype must be F32, BF16 or F16");
  if (H % 4 || s_ym % 4 || s_ot % 4 || !aligned(y, 16) || !aligned(out, 16))
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": rows must start at multiples of 4 elements, 16-byte "
                                                           "aligned, with H % 4 == 0");
  if (ids_dtype != BH_HEX_I32 && ids_dtype != BH_HEX_I64)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": ids dtype must be I32 or I64");
  if (out_dtype != BH_HEX_F32 && out_dtype != BH_HEX_BF16 && out_dtype != BH_HEX_F16)
    return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": out dtype must be F32, BF16 or F16");
  if (T == 0) return BH_HEX_OK;
  if (T > 65535) return fail(BH_HEX_ERR_UNSUPPORTED, std::string(who) + ": more than 65535 tokens");
  const dim3 grid((unsigned)cdiv(H, 1024), (unsigned)T);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define BH_RED(ODT, IDT) reduce_ydt<ODT, IDT>(y_dtype, grid, st, y, s_ym, topk_ids, n_experts, k, H, out, s_ot)
  if (out_dtype == BH_HEX_F32) {
    if (ids_dtype == BH_HEX_I64) BH_RED(BH_HEX_F32, BH_HEX_I64); else BH_RED(BH_HEX_F32, BH_HEX_I32);
  } else if (out_dtype == BH_HEX_BF16) {
    if (ids_dtype == BH_HEX_I64) BH_RED(BH_HEX_BF16, BH_HEX_I64); else BH_RED(BH_HEX_BF16, BH_HEX_I32);
  } else {
    if (ids_dtype == BH_HEX_I64) BH_RED(BH_HEX_F16, BH_HEX_I64); else BH_RED(BH_HEX_F16, BH_HEX_I32);
  }
#undef BH_RED
  return check_launch(who);
}
