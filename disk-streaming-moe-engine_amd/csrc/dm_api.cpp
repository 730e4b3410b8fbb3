// dm_api.cpp -- C ABI of libdismoen_hip.so (include/dismoen_hip.h): context,
// one-time layer upload, and the MoE block entry points.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <chrono>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/dismoen_hip.h"
#include "dm_api_internal.h"
#include <cstdlib>

#include "dm_decode.h"
#include "dm_gguf.h"
#include "dm_grouped.h"
#include "dm_kernels.h"
#include "dm_layout.h"

using dm::LayerDev;

namespace {

constexpr int kMaxLayers = 4096;
constexpr int kMaxDevices = 64;
// Live contexts per device in this process.  The single-launch decode
// kernel needs all its workgroups resident at once; with one context its
// launches are stream-ordered and a plain launch suffices, with several the
// grids of two contexts could each hold part of the device and wait for
// each other, so their launches are cooperative (the runtime then keeps each
// grid whole).
std::atomic<int> g_live_ctx[kMaxDevices];

// Scratch of dmh_moe_forward_noalloc: a file-scope device array, one copy
// per GPU the library runs on, held until the process ends.  Host code never
// uses the array's name as an address: dmh_create resolves each device's
// copy once (hipGetSymbolAddress with that device current) into
// g_scratch_dev[device], and only that pointer reaches kernels.  Every call
// of the entry point on a device shares that device's copy, so the calls on
// one device are put in one order: each call's stream waits for the event
// the previous call (from any context) recorded after its kernels, and
// records it again after its own (g_noalloc_ev, created with the address).
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
void* g_scratch_dev[kMaxDevices];
hipEvent_t g_noalloc_ev[kMaxDevices];
bool g_noalloc_recorded[kMaxDevices];
std::mutex g_scratch_mu;
// first-error key slots: [0, kMaxLayers) uploaded 4-bit layers, kMaxLayers
// the unit calls, then one per GGUF layer
constexpr int kGgufSlot0 = kMaxLayers + 1;
constexpr int kStatusSlots = kGgufSlot0 + kMaxLayers;

// One MoE layer uploaded from a GGUF file: one device block holding the fp32
// router and shared gate, the expert offset table and the expert payloads.
struct GgufLayer {
  dmh_moe_dims dims{};
  void* buf = nullptr;
  size_t bytes = 0;
  dm::GgufMoeDev dev{};
  // single-token form (dm::launch_gguf_one_token): its sync area, grid and
  // launch count (the hand-off count only grows)
  void* sync = nullptr;
  size_t sync_bytes = 0;
  int grid = 0;
  unsigned launches = 0;
  float* rchain = nullptr;  // the router in chain order (dev.rchain)
};

void free_glayer(GgufLayer* G) {
  if (!G) return;
  if (G->buf) (void)hipFree(G->buf);
  if (G->sync) (void)hipFree(G->sync);
  if (G->rchain) (void)hipFree(G->rchain);
  delete G;
}

struct Layer {
  dmh_moe_dims dims{};
  void* buf = nullptr;
  size_t bytes = 0;
  LayerDev dev{};
  bool router_w_bad = false;
  dm::DecodePlan plan{};
  bool fused = false;  // the fused decode kernel fits this layer on this device
  // The fused kernel's counters and tags only grow; launch n of this layer
  // waits for n times the arrivals of one launch (or tag n), so each layer
  // keeps its own hand-off buffers and launch count.
  void* sync = nullptr;
  size_t sync_bytes = 0;
  unsigned launches = 0;
  // post_attention_layernorm gamma [H] fp32 of the block-edge RMSNorm
  // (dmh_set_layer_norm); nullptr: gamma = 1
  float* gamma = nullptr;
};

template <typename T>
struct DevBuf {
  T* p = nullptr;
  size_t cap = 0;  // elements
  hipError_t ensure(size_t n) {
    if (n <= cap) return hipSuccess;
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    hipError_t e = hipMalloc(&p, n * sizeof(T) + 256);
    if (e == hipSuccess) cap = n;
    return e;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
  }
};

// Page-locked host memory for the host-pointer calls (hipHostMalloc): the
// copies are single DMA transfers instead of staged ones, and kernels can
// read and write it directly through its device address d.  flags: the
// single-token call's output block is coherent (fine-grained) memory, so the
// fused decode kernel's stores reach it without staying in the GPU's caches,
// and each workgroup's status key is a system-scope release after its
// outputs: a host that sees the key sees the outputs.  Inputs stay in a
// default block, which the GPU may cache (every workgroup reads all of x).
struct PinBuf {
  uint8_t* p = nullptr;
  uint8_t* d = nullptr;
  size_t cap = 0;  // bytes
  unsigned flags = hipHostMallocDefault;
  hipError_t ensure(size_t n) {
    if (n <= cap) return hipSuccess;
    release();
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&p), n, flags);
    if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void**>(&d), p, 0);
    if (e != hipSuccess) {
      release();
      return e;
    }
    cap = n;
    return hipSuccess;
  }
  void release() {
    if (p) (void)hipHostFree(p);
    p = d = nullptr;
    cap = 0;
  }
};

}  // namespace

struct dmh_ctx {
  int device = 0;
  hipStream_t own = nullptr, cur = nullptr;
  std::vector<Layer*> layers;
  // scratch
  DevBuf<float> x, res, y, z, probs, shg, h, xn, hstack;
  DevBuf<int32_t> ids, uids;  // uids: checked expert ids of dmh_experts_forward
  // host-pointer dmh_moe_forward: inputs [x | residual] and outputs
  // [y | ids | probs | shared gate | status key], one block each on the
  // device and page-locked on the host
  DevBuf<uint8_t> io_in, io_out;
  PinBuf pin;
  PinBuf pin_out{nullptr, nullptr, 0, hipHostMallocCoherent};
  DevBuf<uint8_t> stage;
  // several tokens per call (grouped experts)
  DevBuf<int32_t> g_off, g_perm, g_meta, g_needlo;
  DevBuf<int2> g_units;
  DevBuf<uint16_t> g_xhi, g_xlo;
  DevBuf<uint16_t> g_hr, g_hs;  // bf16 hi parts, then lo parts
  DevBuf<float> g_r, g_rs;
  std::vector<GgufLayer*> glayers;
  unsigned long long* status = nullptr;  // [kStatusSlots] first-error keys
  // status_clean[l]: slot l holds no error and nothing has run on it since
  // a host-pointer call read it back, so the next one need not reset it
  std::vector<uint8_t> status_clean;
  unsigned long long* vkey = nullptr;    // upload validation key
  unsigned* flags = nullptr;             // upload flags
  // where to find the routing of the last device-mode call per layer
  std::vector<const int32_t*> last_ids;
  std::vector<int> last_k;
  int num_cus = 0;
  int xcd_nx = 0;  // XCDs when workgroup b runs on XCD b % xcd_nx (probed), else 0
  bool counted = false;           // counted in g_live_ctx
  float* ones = nullptr;          // [kNormMaxH] 1.0f: gamma of layers without one
  hipEvent_t switch_ev = nullptr;  // orders a stream switch after queued work
  // polls of a persistent kernel's wait before it gives up (dmh_set_spin_limit)
  long spin_limit = dm::kDefaultSpinLimit;
  // host-pointer calls rerun through the multi-kernel path after a time-out
  int64_t sync_fallbacks = 0;
};

namespace {

int set_err(char* err, size_t errlen, int code, const char* fmt, ...) {
  if (err && errlen) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return code;
}

#define HIP_TRY(expr)                                                                      \
  do {                                                                                     \
    hipError_t _e = (expr);                                                                \
    if (_e != hipSuccess)                                                                  \
      return set_err(err, errlen, DMH_ERR_HIP, "{\"error_type\":\"HIP_ERROR\",\"detail\":" \
                     "\"%s: %s\",\"stage\":\"hip\"}", #expr, hipGetErrorString(_e));       \
  } while (0)

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Text of the first error recorded by the kernels (key layout in dm_layout.h).
int decode_key(uint64_t key, int layer, int expert_id, int E, char* err, size_t errlen) {
  using namespace dm;
  const uint32_t ph = key_phase(key), pos = key_pos(key), kind = key_kind(key);
#define RJ(code, type, detail, stage)                                                        \
  return set_err(err, errlen, code,                                                          \
                 "{\"error_type\":\"" type "\",\"detail\":\"" detail "\",\"stage\":\"" stage \
                 "\",\"layer\":%d}", layer)
#define EJ(code, type, detail)                                                              \
  return set_err(err, errlen, code,                                                         \
                 "{\"error_type\":\"" type "\",\"detail\":\"" detail                        \
                 "\",\"stage\":\"swiglu\",\"layer\":%d,\"expert_id\":%d}", layer, expert_id)
  switch (ph) {
    case kPhX: RJ(DMH_ERR_ACT, "ACT_LOAD_FAILED", "non-finite value in activation", "router");
    case kPhRouterW:
      RJ(DMH_ERR_WEIGHT, "WEIGHT_LOAD_FAILED", "non-finite value in router weight", "router");
    case kPhLogit: RJ(DMH_ERR_ROUTER, "ROUTER_ERROR", "non-finite router logit computed", "router");
    case kPhSoftmax:
      if (pos == 0) RJ(DMH_ERR_ROUTER, "ROUTER_ERROR", "non-finite max logit in router softmax", "router");
      if ((int)pos <= E) RJ(DMH_ERR_ROUTER, "ROUTER_ERROR", "non-finite exp in router softmax", "router");
      RJ(DMH_ERR_ROUTER, "ROUTER_ERROR", "invalid sum_exp in router softmax", "router");
    case kPhTopk:
      if (kind == kTkSum)
        RJ(DMH_ERR_ROUTER, "ROUTER_ERROR", "sum of top-k probabilities exceeds 1.0", "router");
      RJ(DMH_ERR_ROUTER, "ROUTER_ERROR",
         "renormalization leak detected: sum of top-k probabilities is 1.0", "router");
    case kPhExpert:
    case kPhShared:
      if (kind == kEkGate) EJ(DMH_ERR_EXPERT, "EXPERT_ERROR", "non-finite in gate projection");
      if (kind == kEkUp) EJ(DMH_ERR_EXPERT, "EXPERT_ERROR", "non-finite in up projection");
      if (kind == kEkH) EJ(DMH_ERR_SWIGLU, "SWIGLU_ERROR", "non-finite in element-wise product");
      if (kind == kEkBadId) {  // the id itself is the key's position (28-bit two's complement)
        expert_id = (int)(pos << 4) >> 4;
        EJ(DMH_ERR_INVALID_ARG, "EXPERT_ERROR", "expert id out of range");
      }
      if (kind == kEkRecheck)
        RJ(DMH_ERR_EXPERT, "EXPERT_ERROR", "non-finite value in aggregation", "aggregation");
      EJ(DMH_ERR_EXPERT, "EXPERT_ERROR", "non-finite in down projection");
    case kPhGate:
      if (kind == kGkLogit) RJ(DMH_ERR_GATE, "GATE_ERROR", "non-finite shared gate logit", "shared");
      RJ(DMH_ERR_GATE, "GATE_ERROR", "shared gate score outside (0, 1)", "shared");
    case kPhSync:
      if (pos == 1)
        RJ(DMH_ERR_HIP, "HIP_ERROR", "decode kernel workgroup ran on an unexpected XCD", "hip");
      return set_err(err, errlen, DMH_ERR_HIP,
                     "{\"error_type\":\"HIP_ERROR\",\"detail\":\"cross-workgroup handoff timed "
                     "out in the decode kernel (wait %u)\",\"stage\":\"hip\",\"layer\":%d}",
                     pos, layer);
    default:
      RJ(DMH_ERR_EXPERT, "EXPERT_ERROR", "non-finite value in aggregation", "aggregation");
  }
#undef RJ
#undef EJ
}

int router_config_check(int E, int K, int norm, char* err, size_t errlen) {
  // RouterConfig.validate, src/layers/router_types.mojo:9-44
  if (E <= 0)
    return set_err(err, errlen, DMH_ERR_CONFIG,
                   "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"num_experts must be"
                   " positive\",\"stage\":\"router\"}");
  if (K <= 0)
    return set_err(err, errlen, DMH_ERR_CONFIG,
                   "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"num_experts_per_tok"
                   " must be positive\",\"stage\":\"router\"}");
  if (K > E)
    return set_err(err, errlen, DMH_ERR_CONFIG,
                   "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"num_experts_per_tok"
                   " cannot exceed num_experts\",\"stage\":\"router\"}");
  if (norm)
    return set_err(err, errlen, DMH_ERR_ROUTER,
                   "{\"error_type\":\"ROUTER_ERROR\",\"detail\":\"norm_topk_prob=true"
                   " forbidden; unrenormalized routing invariant violated\",\"stage\":\"router\"}");
  return DMH_OK;
}

}  // namespace

// The dimensions the 4-bit block supports, checked before any arithmetic
// or allocation that depends on them.  group_size: the reference's allowed
// sizes (src/format/half_float.mojo:24-31, is_allowed_group_size).
int dm::api_moe_dims_check(const dmh_moe_dims* d, int layer, char* err, size_t errlen) {
  const int H = d->hidden, E = d->num_experts, K = d->top_k, I = d->inter, Ish = d->inter_sh;
  const int G = d->group_size;
  const bool g_ok = G == 32 || G == 64 || G == 128 || G == 256;
  if (!g_ok || E <= 0 || K <= 0 || H <= 0 || I <= 0 || Ish <= 0 || H % 128 || I % 128 ||
      Ish % 128 || E > 2048 || K + 1 > 33 || H > 8192 || I > 8192 || Ish > 8192 ||
      (size_t)(K + 1) * (I > Ish ? I : Ish) * 6 > 65536)
    return set_err(err, errlen, DMH_ERR_CONFIG,
                   "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"unsupported MoE dims: G=%d H=%d"
                   " E=%d K=%d I=%d Ish=%d (need G in {32, 64, 128, 256}, H/I/Ish multiples of"
                   " 128, E<=2048, K<=32, H/I/Ish<=8192)\",\"stage\":\"config\",\"layer\":%d}",
                   G, H, E, K, I, Ish, layer);
  return DMH_OK;
}

namespace {

Layer* get_layer(dmh_ctx* ctx, int layer) {
  if (!ctx || layer < 0 || layer >= (int)ctx->layers.size()) return nullptr;
  return ctx->layers[layer];
}

// A first-error key that says a wait between workgroups gave up.
bool sync_timeout(uint64_t key) {
  return key != dm::kNoError && dm::key_phase(key) == dm::kPhSync;
}

hipError_t reset_status(dmh_ctx* ctx, int slot) {
  return hipMemsetAsync(ctx->status + slot, 0xFF, sizeof(unsigned long long), ctx->cur);
}

// Runs the block for T tokens of a layer on device buffers.
hipError_t reset_counters(dmh_ctx* ctx, Layer* Ly) {
  Ly->launches = 0;
  if (!Ly->sync) return hipSuccess;
  return hipMemsetAsync(Ly->sync, 0, Ly->sync_bytes, ctx->cur);
}

void free_layer(Layer* Ly) {
  if (!Ly) return;
  if (Ly->buf) (void)hipFree(Ly->buf);
  if (Ly->sync) (void)hipFree(Ly->sync);
  if (Ly->gamma) (void)hipFree(Ly->gamma);
  delete Ly;
}

// The block-edge norm of a layer: its gamma, or the context's ones.
dm::NormSpec layer_norm(const dmh_ctx* ctx, const Layer* Ly, float eps, bool tree) {
  return dm::NormSpec{eps, Ly->gamma ? Ly->gamma : ctx->ones, tree ? 0 : 1};
}

// Token counts from which the router runs on the matrix cores (bf16
// activations); below it the lane-chain router is as fast.
constexpr int kMfmaRouterMinTokens = 64;
// need-lo flag, then the front end's token counter and per-token counters
constexpr int kFlagInts = 2 + dm::kFrontMaxT + 1;

// Device scratch of one run_block call.  Which buffers a call touches
// depends on its path: the fused decode kernel none of them; the
// multi-kernel single-token path z and h; several tokens z and the g_*
// buffers; xn when the input is normalised outside the fused kernel.
struct BlockScratch {
  float* z = nullptr;         // [T][E+1] logits (and the shared-gate logit)
  float* h = nullptr;         // [K+1][ldh] h of one token
  float* xn = nullptr;        // [T][H] normalised input
  int32_t* off = nullptr;     // [E+1] expert offsets
  int32_t* perm = nullptr;    // [T*K] assignments in expert order
  int32_t* meta = nullptr;    // [2] unit counts
  int32_t* needlo = nullptr;  // [kFlagInts] zero on entry: the need-lo flag (the combine
                              // clears it again) and the front-end arrival counters
                              // (reset by the front-end kernel itself)
  int2* units = nullptr;      // [group_units_max(T, K, E)]
  uint16_t* xhi = nullptr;    // [T][H] bf16 hi parts of x
  uint16_t* xlo = nullptr;    // [T][H] bf16 lo parts
  uint16_t* hr = nullptr;     // [2][T*K][I] routed h, hi then lo
  uint16_t* hs = nullptr;     // [2][T][Ish] shared h, hi then lo
  float* r = nullptr;         // [T*K][H] routed down outputs
  float* rs = nullptr;        // [T][H] shared down outputs
};

// Byte offsets of the scratch of T tokens carved from one block (each
// buffer 256-byte aligned); returns the total.
size_t scratch_carve(const LayerDev& L, int T, bool norm, uint8_t* base, BlockScratch* s) {
  const size_t TK = (size_t)T * L.K, TH = (size_t)T * L.H;
  const size_t ldh = (size_t)(L.I > L.Ish ? L.I : L.Ish);
  size_t off = 0;
  auto take = [&](size_t bytes) -> uint8_t* {
    uint8_t* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  BlockScratch t;
  t.z = (float*)take((size_t)T * (L.E + 1) * 4);
  t.h = (float*)take((size_t)(L.K + 1) * ldh * 4);
  t.xn = norm ? (float*)take(TH * 4) : nullptr;
  if (T > 1) {
    t.off = (int32_t*)take((size_t)(L.E + 1) * 4);
    t.perm = (int32_t*)take(TK * 4);
    t.meta = (int32_t*)take(2 * 4);
    t.needlo = (int32_t*)take(kFlagInts * 4);
    t.units = (int2*)take((size_t)dm::group_units_max(T, L.K, L.E) * sizeof(int2));
    t.xhi = (uint16_t*)take(TH * 2);
    t.xlo = (uint16_t*)take(TH * 2);
    t.hr = (uint16_t*)take(2 * TK * L.I * 2);
    t.hs = (uint16_t*)take(2 * (size_t)T * L.Ish * 2);
    t.r = (float*)take(TK * L.H * 4);
    t.rs = (float*)take(TH * 4);
  }
  if (s) *s = t;
  return off;
}

// The scratch of a call from the context's buffers, grown on demand (the
// need-lo flag is zeroed when it is allocated and cleared by the combine
// kernel that ends every call).
hipError_t ctx_scratch(dmh_ctx* ctx, const LayerDev& L, int T, bool norm, BlockScratch* s) {
  const size_t TK = (size_t)T * L.K, TH = (size_t)T * L.H;
  const int ldh = L.I > L.Ish ? L.I : L.Ish;
  hipError_t e;
  if (norm) {
    if ((e = ctx->xn.ensure(TH)) != hipSuccess) return e;
    s->xn = ctx->xn.p;
  }
  if ((e = ctx->z.ensure((size_t)T * (L.E + 1))) != hipSuccess) return e;
  if ((e = ctx->h.ensure((size_t)(L.K + 1) * ldh)) != hipSuccess) return e;
  s->z = ctx->z.p;
  s->h = ctx->h.p;
  if (T <= 1) return hipSuccess;
  if ((e = ctx->g_off.ensure(L.E + 1)) != hipSuccess) return e;
  if ((e = ctx->g_perm.ensure(TK)) != hipSuccess) return e;
  if ((e = ctx->g_meta.ensure(2)) != hipSuccess) return e;
  const size_t nl_cap = ctx->g_needlo.cap;
  if ((e = ctx->g_needlo.ensure(kFlagInts)) != hipSuccess) return e;
  if (ctx->g_needlo.cap != nl_cap &&
      (e = hipMemsetAsync(ctx->g_needlo.p, 0, kFlagInts * sizeof(int), ctx->cur)) != hipSuccess)
    return e;
  if ((e = ctx->g_units.ensure(dm::group_units_max(T, L.K, L.E))) != hipSuccess) return e;
  if ((e = ctx->g_xhi.ensure(TH)) != hipSuccess) return e;
  if ((e = ctx->g_xlo.ensure(TH)) != hipSuccess) return e;
  if ((e = ctx->g_hr.ensure(2 * TK * L.I)) != hipSuccess) return e;
  if ((e = ctx->g_hs.ensure(2 * (size_t)T * L.Ish)) != hipSuccess) return e;
  if ((e = ctx->g_r.ensure(TK * L.H)) != hipSuccess) return e;
  if ((e = ctx->g_rs.ensure(TH)) != hipSuccess) return e;
  s->off = ctx->g_off.p;
  s->perm = ctx->g_perm.p;
  s->meta = ctx->g_meta.p;
  s->needlo = ctx->g_needlo.p;
  s->units = ctx->g_units.p;
  s->xhi = ctx->g_xhi.p;
  s->xlo = ctx->g_xlo.p;
  s->hr = ctx->g_hr.p;
  s->hs = ctx->g_hs.p;
  s->r = ctx->g_r.p;
  s->rs = ctx->g_rs.p;
  return hipSuccess;
}

// nm (may be NULL): the block's input is rmsnorm(dx, nm->gamma, nm->eps),
// computed inside the fused decode kernel or by a separate kernel into
// scratch xn.  sc (may be NULL): the scratch to use instead of the
// context's buffers.  Under stream capture the fused kernel is not used: its
// launch tag is fixed on the host, so every replay of a captured launch
// would carry the same tag and its waits would pass on the previous replay's
// data.
constexpr int kTokMinT = 3;  // fewest tokens of the several-token launch

hipError_t run_block(dmh_ctx* ctx, Layer* Ly, int layer, const float* dx, const float* dres,
                     int T, float* dy, int32_t* dids, float* dprobs, float* dshg,
                     bool allow_fused = true, const dm::NormSpec* nm = nullptr,
                     const BlockScratch* sc = nullptr, unsigned long long* status_out = nullptr,
                     bool* exported = nullptr) {
  const LayerDev& L = Ly->dev;
  hipStream_t st = ctx->cur;
  unsigned long long* status = ctx->status + layer;
  ctx->status_clean[layer] = 0;
  const int ldh = L.I > L.Ish ? L.I : L.Ish;
  hipError_t e;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if ((e = hipStreamIsCapturing(st, &cap)) != hipSuccess) return e;
  const bool fused = Ly->fused && allow_fused && T == 1 && cap == hipStreamCaptureStatusNone;
  const dm::NormSpec no_norm{0.0f, nullptr, 0};
  const bool norm = nm && nm->eps > 0.0f;
  if (Ly->fused && allow_fused && cap == hipStreamCaptureStatusNone && !norm &&
      T >= kTokMinT && T <= dm::kTokMaxT && Ly->plan.tok && T <= Ly->plan.xs_nx) {
    // a few tokens: each one's whole block on one XCD, in one launch (from
    // three tokens on: with two, six XCDs would idle and the grouped path
    // measured as fast)
    if (Ly->launches >= (1u << 24) && (e = reset_counters(ctx, Ly)) != hipSuccess) return e;
    dm::DecodeSync S = dm::decode_sync_carve(L, Ly->plan, Ly->sync);
    S.n = ++Ly->launches;
    S.spin = ctx->spin_limit;
    S.trace = layer;
    return dm::launch_moe_tokens(L, Ly->plan, dx, T, dres, dy, dids, dprobs, dshg, S, status, st,
                                 g_live_ctx[ctx->device].load(std::memory_order_relaxed) > 1);
  }
  if (fused) {
    for (int t = 0; t < T; ++t) {
      if (Ly->launches >= (1u << 24) && (e = reset_counters(ctx, Ly)) != hipSuccess) return e;
      dm::DecodeSync S = dm::decode_sync_carve(L, Ly->plan, Ly->sync);
      S.n = ++Ly->launches;
      S.spin = ctx->spin_limit;
      S.trace = layer;
      e = dm::launch_moe_decode(L, Ly->plan, dx + (size_t)t * L.H,
                                dres ? dres + (size_t)t * L.H : nullptr, dy + (size_t)t * L.H,
                                dids + (size_t)t * L.K, dprobs + (size_t)t * L.K, dshg + t, S,
                                status, t, st, norm ? *nm : no_norm,
                                g_live_ctx[ctx->device].load(std::memory_order_relaxed) > 1,
                                status_out);
      if (e != hipSuccess) return e;
    }
    if (exported) *exported = status_out != nullptr;
    return hipSuccess;
  }
  BlockScratch own;
  if (!sc) {
    if ((e = ctx_scratch(ctx, L, T, norm, &own)) != hipSuccess) return e;
    sc = &own;
  }
  if (norm) {
    if ((e = dm::launch_rmsnorm_rows(dx, T, L.H, *nm, sc->xn, st)) != hipSuccess) return e;
    dx = sc->xn;
  }
  if (T > 1) {
    // several tokens: route, group the assignments by expert and run each
    // expert's tokens together as a grouped GEMM
    const size_t TK = (size_t)T * L.K, TH = (size_t)T * L.H;
    if (T < kMfmaRouterMinTokens && dm::front_supported(L, T)) {
      // split, router, selection and grouping in one launch
      if ((e = dm::launch_front(L, dx, T, sc->z, sc->xhi, sc->xlo, sc->needlo, dids, dprobs, dshg,
                                sc->off, sc->perm, sc->units, sc->meta, status, st)) !=
          hipSuccess)
        return e;
      if ((e = dm::launch_experts_grouped(L, sc->xhi, sc->xlo, sc->needlo, sc->off, sc->perm,
                                          sc->units, sc->meta, T, sc->hr, sc->hr + TK * L.I,
                                          sc->hs, sc->hs + (size_t)T * L.Ish, sc->r, sc->rs,
                                          status, st)) != hipSuccess)
        return e;
      return dm::launch_combine(sc->r, sc->rs, dprobs, dshg, dres, T, L.H, L.K, dy, status, st,
                                sc->needlo);
    }
    if ((e = dm::launch_split_rows(dx, (int64_t)TH, sc->xhi, sc->xlo, sc->needlo, st)) !=
        hipSuccess)
      return e;
    if (T >= kMfmaRouterMinTokens) {
      // bf16 activations: matrix-core router; otherwise the lane-chain router
      if ((e = dm::launch_router_mfma(L, sc->xhi, sc->needlo, T, sc->z, st)) != hipSuccess)
        return e;
      if ((e = dm::launch_router_dec(L, dx, T, sc->z, status, st, sc->needlo)) != hipSuccess)
        return e;
    } else if ((e = dm::launch_router_dec(L, dx, T, sc->z, status, st)) != hipSuccess) {
      return e;
    }
    if ((e = dm::launch_router_select(sc->z, L.E + 1, T, L.E, L.K, 1, dids, dprobs, dshg,
                                      status, st)) != hipSuccess)
      return e;
    if ((e = dm::launch_group_build(dids, T, L.K, L.E, sc->off, sc->perm, sc->units, sc->meta,
                                    st)) != hipSuccess)
      return e;
    if ((e = dm::launch_experts_grouped(L, sc->xhi, sc->xlo, sc->needlo, sc->off, sc->perm,
                                        sc->units, sc->meta, T, sc->hr, sc->hr + TK * L.I, sc->hs,
                                        sc->hs + (size_t)T * L.Ish, sc->r, sc->rs, status, st)) !=
        hipSuccess)
      return e;
    return dm::launch_combine(sc->r, sc->rs, dprobs, dshg, dres, T, L.H, L.K, dy, status, st,
                              sc->needlo);
  }
  if ((e = dm::launch_router_dec(L, dx, T, sc->z, status, st)) != hipSuccess) return e;
  if ((e = dm::launch_router_select(sc->z, L.E + 1, T, L.E, L.K, 1, dids, dprobs, dshg, status,
                                    st)) != hipSuccess)
    return e;
  for (int t = 0; t < T; ++t) {
    const float* xt = dx + (size_t)t * L.H;
    if ((e = dm::launch_gateup_dec(L, xt, dids + (size_t)t * L.K, sc->h, ldh, t, status, st)) !=
        hipSuccess)
      return e;
    if ((e = dm::launch_down_dec(L, sc->h, ldh, dids + (size_t)t * L.K,
                                 dprobs + (size_t)t * L.K, dshg + t,
                                 dres ? dres + (size_t)t * L.H : nullptr, dy + (size_t)t * L.H, t,
                                 status, st)) != hipSuccess)
      return e;
  }
  return hipSuccess;
}

// Host-side decode of a layer's status word after a synchronous call.
int finish_status(dmh_ctx* ctx, Layer* Ly, int layer, uint64_t key, const int32_t* host_ids,
                  char* err, size_t errlen, int ids_k = 0) {
  if (Ly && Ly->router_w_bad) {
    const uint64_t rk = dm::err_key(dm::kPhRouterW, 0, 0, 0, 0);
    if (rk < key) key = rk;
  }
  if (key == dm::kNoError) return DMH_OK;
  if (dm::key_phase(key) == dm::kPhSync && Ly) {
    (void)hipStreamSynchronize(ctx->cur);
    (void)reset_counters(ctx, Ly);
  }
  int expert_id = -1;
  const int K = ids_k > 0 ? ids_k : Ly ? Ly->dims.top_k : 0;
  if (dm::key_phase(key) == dm::kPhExpert && host_ids)
    expert_id = host_ids[(size_t)dm::key_token(key) * K + dm::key_slot(key)];
  return decode_key(key, layer, expert_id, Ly ? Ly->dims.num_experts : 0, err, errlen);
}

// The error text of a GGUF layer's first-error key.  forward_port_block
// calls swiglu_forward(x, w, seq_len, hidden, inter) (port_scheduler.mojo:
// 450-464), so the expert texts carry hidden as the layer and the
// intermediate size as the expert id.
int gguf_finish(dmh_ctx* c, int layer, uint64_t key, char* err, size_t errlen) {
  GgufLayer* G = layer >= 0 && layer < (int)c->glayers.size() ? c->glayers[layer] : nullptr;
  const int H = G ? G->dims.hidden : 0, E = G ? G->dims.num_experts : 0;
  const uint32_t ph = dm::key_phase(key);
  if (ph == dm::kPhSync && G && G->sync) {  // a hand-off timed out: start the count again
    (void)hipStreamSynchronize(c->cur);
    if (hipMemsetAsync(G->sync, 0, G->sync_bytes, c->cur) == hipSuccess) G->launches = 0;
  }
  if (ph == dm::kPhExpert || ph == dm::kPhShared)
    return decode_key(key, H, ph == dm::kPhShared ? (G ? G->dims.inter_sh : 0)
                                                   : (G ? G->dims.inter : 0),
                      E, err, errlen);
  return decode_key(key, layer, -1, E, err, errlen);
}

GgufLayer* get_glayer(dmh_ctx* c, int layer) {
  if (!c || layer < 0 || layer >= (int)c->glayers.size()) return nullptr;
  return c->glayers[layer];
}

// The MoE section of forward_port_block on a GGUF layer, all on the device:
// one token in one launch (dm::launch_gguf_one_token) when the layer has
// its sync area, no other context of the library lives on the device (its
// persistent grids could hold CUs the launch waits for) and the
// stream is not being captured (a replay would repeat the launch count);
// otherwise router and shared-gate logits (fp32 weights, router_forward's
// order), selection and gate, then from kGgufGroupMinT tokens on the
// grouping by expert and the grouped gate/up, down and combine launches
// (dm::launch_gguf_units), below it gate/up of every (token, slot) and the
// down projections with moe_aggregate_forward.
// The grouped several-token form: from 128 tokens on (below, the units hold
// one or two tokens and the grid sized for the most units there could be
// costs more than the rows it saves: Qwen3.6 shape, Q3_K, per call 851
// against 957 us at 128 tokens, 404 against 258 at 32), for at most 4096
// experts (the grouping's LDS holds two ints per expert).
constexpr int kGgufGroupMinT = 128;
constexpr int kGgufGroupMaxE = 4096;

hipError_t run_gguf_block(dmh_ctx* c, GgufLayer* G, unsigned long long* status, const float* dx,
                          const float* dres, int T, float* dy, int32_t* dids, float* dprobs,
                          float* dshg, bool allow_one = true) {
  const dm::GgufMoeDev& L = G->dev;
  hipStream_t st = c->cur;
  hipError_t e;
  if (allow_one && T == 1 && G->sync && G->grid > 0 &&
      g_live_ctx[c->device].load(std::memory_order_relaxed) <= 1) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(st, &cap)) != hipSuccess) return e;
    if (cap == hipStreamCaptureStatusNone) {
      if (G->launches >= (1u << 24)) {
        if ((e = hipMemsetAsync(G->sync, 0, G->sync_bytes, st)) != hipSuccess) return e;
        G->launches = 0;
      }
      return dm::launch_gguf_one_token(L, dx, dres, dy, dids, dprobs, dshg, G->sync,
                                       ++G->launches, G->grid, status, st, c->spin_limit);
    }
  }
  const int ldh = L.I > L.Ish ? L.I : L.Ish;
  if ((e = c->z.ensure((size_t)T * (L.E + 1))) != hipSuccess) return e;
  if ((e = c->h.ensure((size_t)T * (L.K + 1) * ldh)) != hipSuccess) return e;
  // router logits and, as column E, the shared-gate logit in the same
  // 16-lane order; the selection kernel applies the gate's sigmoid and its
  // GATE_ERROR checks
  const int rs = (int)(dm::gguf_chain_router_bytes(L) / ((size_t)(L.E + 1) * sizeof(float)));
  if (L.rchain && dm::router_rows_f32_ok(T, L.H, L.E, rs)) {
    // many tokens: the chain-ordered copy, four tokens per pass (the same bits)
    if ((e = dm::launch_router_rows_f32(dx, L.rchain, rs, T, L.H, L.E, c->z.p, status, st)) !=
        hipSuccess)
      return e;
  } else if ((e = dm::launch_router_generic(dx, L.router, T, L.H, L.E, c->z.p, status, st,
                                            L.shgate)) != hipSuccess) {
    return e;
  }
  if ((e = dm::launch_router_select(c->z.p, L.E + 1, T, L.E, L.K, 1, dids, dprobs, dshg, status,
                                    st)) != hipSuccess)
    return e;
  if (T >= kGgufGroupMinT && L.E <= kGgufGroupMaxE) {
    // several tokens: grouped by expert, each expert row read once per unit
    const int nu = dm::group_units_max(T, L.K, L.E);
    if ((e = c->g_off.ensure(L.E + 1)) != hipSuccess) return e;
    if ((e = c->g_perm.ensure((size_t)T * L.K)) != hipSuccess) return e;
    if ((e = c->g_meta.ensure(2)) != hipSuccess) return e;
    if ((e = c->g_units.ensure(nu)) != hipSuccess) return e;
    if ((e = c->g_r.ensure((size_t)T * (L.K + 1) * L.H)) != hipSuccess) return e;
    if ((e = dm::launch_group_build(dids, T, L.K, L.E, c->g_off.p, c->g_perm.p, c->g_units.p,
                                    c->g_meta.p, st)) != hipSuccess)
      return e;
    return dm::launch_gguf_units(L, dx, T, c->g_off.p, c->g_perm.p, c->g_units.p, c->g_meta.p, nu,
                                 c->h.p, ldh, c->g_r.p, dprobs, dshg, dres, dy, status, st);
  }
  if ((e = dm::launch_gguf_gateup(L, dx, T, dids, c->h.p, ldh, status, st)) != hipSuccess) return e;
  return dm::launch_gguf_down_combine(L, c->h.p, ldh, T, dids, dprobs, dshg, dres, dy, status,
                                      st);
}

}  // namespace

extern "C" {

const char* dmh_version(void) { return "dismoen_hip 1 gfx950"; }

int dmh_set_spin_limit(dmh_ctx* c, int64_t polls) {
  if (!c) return DMH_ERR_INVALID_ARG;
  c->spin_limit = polls >= 0 ? (long)polls : dm::kDefaultSpinLimit;
  return DMH_OK;
}

int dmh_xcd_rotation(const uint32_t* xcd_of_workgroup, int num_workgroups) {
  return dm::xcd_rotation(xcd_of_workgroup, num_workgroups);
}

int dmh_sync_fallbacks(dmh_ctx* c, int64_t* count) {
  if (!c || !count) return DMH_ERR_INVALID_ARG;
  *count = c->sync_fallbacks;
  return DMH_OK;
}

int dmh_create(int device, dmh_ctx** out, char* err, size_t errlen) {
  if (!out) return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_create: out is NULL");
  *out = nullptr;
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_create: no HIP device %d (%d present)",
                   device, n);
  if (device >= kMaxDevices)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_create: device %d >= %d", device,
                   kMaxDevices);
  HIP_TRY(hipSetDevice(device));
  dmh_ctx* c = new dmh_ctx();
  c->device = device;
  hipError_t e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&c->status, sizeof(unsigned long long) * kStatusSlots);
  if (e == hipSuccess) e = hipMalloc(&c->vkey, sizeof(unsigned long long));
  if (e == hipSuccess) e = hipMalloc(&c->flags, sizeof(unsigned));
  if (e == hipSuccess)
    e = hipMemset(c->status, 0xFF, sizeof(unsigned long long) * kStatusSlots);
  if (e == hipSuccess) e = hipMalloc(&c->ones, sizeof(float) * dm::kNormMaxH);
  if (e == hipSuccess) {
    const std::vector<float> one(dm::kNormMaxH, 1.0f);
    e = hipMemcpy(c->ones, one.data(), sizeof(float) * one.size(), hipMemcpyHostToDevice);
  }
  if (e == hipSuccess) e = hipEventCreateWithFlags(&c->switch_ev, hipEventDisableTiming);
  if (e != hipSuccess) {
    dmh_destroy(c);
    return set_err(err, errlen, DMH_ERR_HIP, "dmh_create: %s", hipGetErrorString(e));
  }
  c->cur = c->own;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->num_cus = prop.multiProcessorCount;
  // where the dispatcher spreads a grid over the XCDs in rotation, the
  // decode kernel can keep hand-offs inside one XCD (its XCD-sliced form);
  // DMH_NO_XCD_SLICING set in the environment keeps the original form
  if (std::getenv("DMH_NO_XCD_SLICING") == nullptr &&
      dm::probe_xcd_map(c->num_cus, &c->xcd_nx) != hipSuccess)
    c->xcd_nx = 0;
  c->last_ids.assign(kMaxLayers + 1, nullptr);
  c->last_k.assign(kMaxLayers + 1, 0);
  c->status_clean.assign(kMaxLayers, 0);
  c->glayers.assign(kMaxLayers, nullptr);
  {
    // this device's copy of the no-allocation scratch, resolved once
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_dev[device]) {
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        dmh_destroy(c);
        return set_err(err, errlen, DMH_ERR_HIP, "dmh_create: scratch address: %s",
                       hipGetErrorString(e));
      }
      hipEvent_t ev = nullptr;
      e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (e != hipSuccess) {
        dmh_destroy(c);
        return set_err(err, errlen, DMH_ERR_HIP, "dmh_create: scratch event: %s",
                       hipGetErrorString(e));
      }
      g_noalloc_ev[device] = ev;
      g_scratch_dev[device] = p;
    }
  }
  g_live_ctx[device].fetch_add(1);
  c->counted = true;
  *out = c;
  return DMH_OK;
}

int dmh_destroy(dmh_ctx* c) {
  if (!c) return DMH_OK;
  (void)hipSetDevice(c->device);
  if (c->cur) (void)hipStreamSynchronize(c->cur);
  for (Layer* L : c->layers) free_layer(L);
  for (GgufLayer* G : c->glayers) free_glayer(G);
  DevBuf<float>* fb[] = {&c->x, &c->res, &c->y, &c->z, &c->probs, &c->shg, &c->h, &c->xn, &c->hstack};
  for (auto* b : fb) b->release();
  c->ids.release();
  c->uids.release();
  c->io_in.release();
  c->io_out.release();
  c->pin.release();
  c->pin_out.release();
  c->stage.release();
  c->g_off.release();
  c->g_perm.release();
  c->g_meta.release();
  c->g_needlo.release();
  c->g_units.release();
  c->g_xhi.release();
  c->g_xlo.release();
  c->g_hr.release();
  c->g_hs.release();
  c->g_r.release();
  c->g_rs.release();
  if (c->status) (void)hipFree(c->status);
  if (c->ones) (void)hipFree(c->ones);
  if (c->switch_ev) (void)hipEventDestroy(c->switch_ev);
  if (c->vkey) (void)hipFree(c->vkey);
  if (c->flags) (void)hipFree(c->flags);
  if (c->own) (void)hipStreamDestroy(c->own);
  if (c->counted) g_live_ctx[c->device].fetch_sub(1);
  delete c;
  return DMH_OK;
}

// Work queued on the old stream is ordered before everything issued on the
// new one (an event recorded on the old stream, waited for by the new), so
// two launches of one layer never interleave their hand-off words.
int dmh_set_stream(dmh_ctx* c, void* s) {
  if (!c) return DMH_ERR_INVALID_ARG;
  hipStream_t nx = s ? (hipStream_t)s : c->own;
  if (nx == c->cur) return DMH_OK;
  if (hipSetDevice(c->device) != hipSuccess || hipEventRecord(c->switch_ev, c->cur) != hipSuccess ||
      hipStreamWaitEvent(nx, c->switch_ev, 0) != hipSuccess)
    return DMH_ERR_HIP;
  c->cur = nx;
  return DMH_OK;
}

void* dmh_get_stream(dmh_ctx* c) { return c ? (void*)c->cur : nullptr; }

int dmh_sync(dmh_ctx* c, char* err, size_t errlen) {
  if (!c) return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_sync: ctx is NULL");
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipStreamSynchronize(c->cur));
  std::vector<unsigned long long> keys(kStatusSlots);
  HIP_TRY(hipMemcpy(keys.data(), c->status, sizeof(unsigned long long) * keys.size(),
                    hipMemcpyDeviceToHost));
  int rc = DMH_OK;
  for (int l = kGgufSlot0; l < kStatusSlots && rc == DMH_OK; ++l)
    if (keys[l] != dm::kNoError) rc = gguf_finish(c, l - kGgufSlot0, keys[l], err, errlen);
  for (int l = 0; l <= kMaxLayers && rc == DMH_OK; ++l) {
    Layer* Ly = l < (int)c->layers.size() ? c->layers[l] : nullptr;
    uint64_t key = keys[l];
    if (key == dm::kNoError) continue;
    std::vector<int32_t> ids;
    const int idk = c->last_k[l] > 0 ? c->last_k[l] : Ly ? Ly->dims.top_k : 0;
    if (dm::key_phase(key) == dm::kPhExpert && c->last_ids[l] && Ly) {
      const size_t n = (size_t)(dm::key_token(key) + 1) * idk;
      ids.resize(n);
      if (hipMemcpy(ids.data(), c->last_ids[l], n * sizeof(int32_t), hipMemcpyDeviceToHost) !=
          hipSuccess)
        ids.clear();
    }
    rc = finish_status(c, Ly, l, key, ids.empty() ? nullptr : ids.data(), err, errlen, idk);
  }
  HIP_TRY(hipMemset(c->status, 0xFF, sizeof(unsigned long long) * keys.size()));
  return rc;
}

int dmh_upload_moe_layer(dmh_ctx* c, int layer, const dmh_moe_dims* d, const dmh_moe_weights* w,
                         unsigned flags, char* err, size_t errlen) {
  if (!c || !d || !w)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_upload_moe_layer: NULL argument");
  if (layer < 0 || layer >= kMaxLayers)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_upload_moe_layer: layer %d outside [0, %d)", layer, kMaxLayers);
  int rc = router_config_check(d->num_experts, d->top_k, d->norm_topk_prob, err, errlen);
  if (rc) return rc;
  const int H = d->hidden, E = d->num_experts, K = d->top_k, I = d->inter, Ish = d->inter_sh;
  if ((rc = dm::api_moe_dims_check(d, layer, err, errlen)) != DMH_OK) return rc;
  if (!w->router_bf16 || !w->shgate_bf16 || !w->gu_scales || !w->gu_packed || !w->d_scales ||
      !w->d_packed || !w->sh_gu_scales || !w->sh_gu_packed || !w->sh_d_scales || !w->sh_d_packed)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_upload_moe_layer: NULL weight pointer");
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->cur;
  // G: one scale per 32 columns on the device; Gs: the source group size
  const size_t G = 32, Gs = (size_t)d->group_size;
  const size_t n_gu = (size_t)E * 2 * I * H, n_d = (size_t)E * H * I;
  const size_t n_sgu = (size_t)2 * Ish * H, n_sd = (size_t)H * Ish;
  // device layout sizes
  const size_t b_router = align256((size_t)(E + 1) * H * 2);
  const size_t b_gun = align256(n_gu / 2), b_gus = align256(n_gu / G * 2);
  const size_t b_dn = align256(n_d / 2), b_ds = align256(n_d / G * 2);
  const size_t b_sgun = align256(n_sgu / 2), b_sgus = align256(n_sgu / G * 2);
  const size_t b_sdn = align256(n_sd / 2), b_sds = align256(n_sd / G * 2);
  const size_t total = b_router + b_gun + b_gus + b_dn + b_ds + b_sgun + b_sgus + b_sdn + b_sds;
  Layer* Ly = new Layer();
  Ly->dims = *d;
  hipError_t e = hipMalloc(&Ly->buf, total);
  if (e != hipSuccess) {
    delete Ly;
    return set_err(err, errlen, DMH_ERR_NO_MEMORY, "dmh_upload_moe_layer: hipMalloc(%zu): %s",
                   total, hipGetErrorString(e));
  }
  Ly->bytes = total;
  uint8_t* p = (uint8_t*)Ly->buf;
  uint16_t* router = (uint16_t*)p; p += b_router;
  uint8_t* gun = p; p += b_gun;
  uint16_t* gus = (uint16_t*)p; p += b_gus;
  uint8_t* dn = p; p += b_dn;
  uint16_t* ds = (uint16_t*)p; p += b_ds;
  uint8_t* sgun = p; p += b_sgun;
  uint16_t* sgus = (uint16_t*)p; p += b_sgus;
  uint8_t* sdn = p; p += b_sdn;
  uint16_t* sds = (uint16_t*)p; p += b_sds;
  Ly->dev = LayerDev{H, E, K, I, Ish, router, gun, gus, dn, ds, sgun, sgus, sdn, sds};

  auto fail = [&](int code, const char* what, hipError_t he) {
    (void)hipFree(Ly->buf);
    delete Ly;
    return set_err(err, errlen, code, "dmh_upload_moe_layer: %s: %s", what, hipGetErrorString(he));
  };
  e = hipMemsetAsync(c->vkey, 0xFF, sizeof(unsigned long long), st);
  if (e == hipSuccess) e = hipMemsetAsync(c->flags, 0, sizeof(unsigned), st);
  if (e != hipSuccess) return fail(DMH_ERR_HIP, "memset", e);

  const bool dev = flags & DMH_F_DEVICE;
  // staging: one tensor group (scales + codes) at a time, sized for the
  // largest of the four groups (the shared expert can outgrow the routed
  // ones), and for the router and shared gate
  size_t stage_bytes = 2 * b_router;
  for (size_t n : {n_gu, n_d, n_sgu, n_sd})
    stage_bytes = std::max(stage_bytes, align256(n / 2) + align256(n / Gs * 2));
  if (!dev && (e = c->stage.ensure(stage_bytes)) != hipSuccess)
    return fail(DMH_ERR_NO_MEMORY, "staging", e);
  auto src = [&](const void* hp, size_t bytes, size_t off, const void** dp) -> hipError_t {
    if (dev) {
      *dp = hp;
      return hipSuccess;
    }
    *dp = c->stage.p + off;
    return hipMemcpyAsync(c->stage.p + off, hp, bytes, hipMemcpyHostToDevice, st);
  };
  const void *s_nib, *s_sc, *s_r, *s_g;
  // router + shared gate
  if ((e = src(w->router_bf16, (size_t)E * H * 2, 0, &s_r)) != hipSuccess ||
      (e = src(w->shgate_bf16, (size_t)H * 2, b_router, &s_g)) != hipSuccess ||
      (e = dm::launch_repack_router((const uint16_t*)s_r, (const uint16_t*)s_g, router, E, H,
                                    c->flags, st)) != hipSuccess)
    return fail(DMH_ERR_HIP, "router upload", e);
  if (!dev && (e = hipStreamSynchronize(st)) != hipSuccess) return fail(DMH_ERR_HIP, "sync", e);
  struct Mat {
    const uint8_t* nib;
    const uint16_t* sc;
    size_t n;
    int R, C, nmat, tbase, per;
    uint8_t* dn;
    uint16_t* ds;
  } mats[] = {
      {w->gu_packed, w->gu_scales, n_gu, I, H, 2 * E, 0, 2, gun, gus},
      {w->d_packed, w->d_scales, n_d, H, I, E, 2, 1, dn, ds},
      {w->sh_gu_packed, w->sh_gu_scales, n_sgu, Ish, H, 2, 3 * E, 2, sgun, sgus},
      {w->sh_d_packed, w->sh_d_scales, n_sd, H, Ish, 1, 3 * E + 2, 1, sdn, sds},
  };
  for (const Mat& m : mats) {
    if ((e = src(m.nib, m.n / 2, 0, &s_nib)) != hipSuccess ||
        (e = src(m.sc, m.n / Gs * 2, align256(m.n / 2), &s_sc)) != hipSuccess)
      return fail(DMH_ERR_HIP, "weight copy", e);
    // per-matrix launches keep the tensor index of the validation key in the
    // reference's load order (gate, up, down of expert 0, then expert 1, ...)
    const size_t mn = (size_t)m.R * m.C;
    for (int i = 0; i < m.nmat; ++i) {
      const int tens = m.tbase + (i / m.per) * 3 + (i % m.per);
      e = dm::launch_repack_a16((const uint8_t*)s_nib + i * (mn / 2),
                                (const uint16_t*)s_sc + i * (mn / Gs), m.dn + i * (mn / 2),
                                m.ds + i * (mn / G), m.R, m.C, 1, tens, (int)Gs, c->vkey, st);
      if (e != hipSuccess) return fail(DMH_ERR_HIP, "repack", e);
    }
    if (!dev && (e = hipStreamSynchronize(st)) != hipSuccess) return fail(DMH_ERR_HIP, "sync", e);
  }
  unsigned long long vk = 0;
  unsigned fl = 0;
  if ((e = hipMemcpyAsync(&vk, c->vkey, sizeof(vk), hipMemcpyDeviceToHost, st)) != hipSuccess ||
      (e = hipMemcpyAsync(&fl, c->flags, sizeof(fl), hipMemcpyDeviceToHost, st)) != hipSuccess ||
      (e = hipStreamSynchronize(st)) != hipSuccess)
    return fail(DMH_ERR_HIP, "validation readback", e);
  if (vk != dm::kNoError) {
    (void)hipFree(Ly->buf);
    delete Ly;
    const uint64_t sub = vk & ((1ull << 34) - 1);
    if (sub & (1ull << 33))
      return set_err(err, errlen, DMH_ERR_DEQUANT,
                     "dequant_kernel: reserved nibble 0b1000 (-8) encountered");
    if (sub & 1ull)
      return set_err(err, errlen, DMH_ERR_DEQUANT,
                     "dequant_kernel: scale is non-positive at group %llu",
                     (unsigned long long)(sub >> 1));
    return set_err(err, errlen, DMH_ERR_DEQUANT, "dequant_kernel: scale is NaN or Inf at group %llu",
                   (unsigned long long)(sub >> 1));
  }
  Ly->router_w_bad = fl & 1u;
  // fused decode kernel: all workgroups must be co-resident
  Ly->plan = dm::make_decode_plan(Ly->dev, c->num_cus, c->xcd_nx);
  {
    int per_cu = 0;
    Ly->sync_bytes = dm::decode_sync_bytes(Ly->dev, Ly->plan);
    if (dm::decode_occupancy(Ly->dev, Ly->plan, &per_cu) == hipSuccess && c->num_cus > 0 &&
        per_cu * c->num_cus >= Ly->plan.grid && Ly->plan.lds_bytes <= 65536 && K + 1 <= 64 &&
        hipMalloc(&Ly->sync, Ly->sync_bytes) == hipSuccess &&
        hipMemsetAsync(Ly->sync, 0, Ly->sync_bytes, st) == hipSuccess)
      Ly->fused = true;
  }
  if (layer >= (int)c->layers.size()) c->layers.resize(layer + 1, nullptr);
  if (c->layers[layer]) {
    (void)hipStreamSynchronize(st);
    free_layer(c->layers[layer]);
  }
  c->layers[layer] = Ly;
  return DMH_OK;
}

int dmh_free_layer(dmh_ctx* c, int layer) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly) return DMH_ERR_INVALID_ARG;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->cur);
  free_layer(Ly);
  c->layers[layer] = nullptr;
  return DMH_OK;
}

int dmh_layer_bytes(dmh_ctx* c, int layer, int64_t* bytes) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly || !bytes) return DMH_ERR_INVALID_ARG;
  *bytes = (int64_t)Ly->bytes;
  return DMH_OK;
}

}  // extern "C"

namespace {

// One token with host pointers, the drop-in's decode call.  The kernels read
// x and the residual from, and write y, ids, probs and the shared gate into,
// the page-locked block through its device address, so the call is one
// launch and one synchronisation (every workgroup of the fused kernel stores
// the status key into the block as it ends, the call's key is their
// minimum; other paths read it back), and the key's reset is skipped while
// the previous host call left it clean.
// A status word no workgroup writes (phase 15 is no phase; only the
// no-error key, all ones, has it).
constexpr unsigned long long kKeySentinel = 0xFFFFFFFFFFFFFFF0ull;
constexpr std::chrono::milliseconds kHostPollLimit{200};

int moe_forward_host1(dmh_ctx* c, Layer* Ly, int layer, const float* x, const float* residual,
                      float* y, int32_t* ids, float* probs, float* shg, const dm::NormSpec* nm,
                      char* err, size_t errlen) {
  const LayerDev& L = Ly->dev;
  const size_t H = (size_t)L.H, K = (size_t)L.K;
  // inputs [x | residual] in one block, outputs [y | ids | probs | shared
  // gate | status keys] in the coherent one
  const size_t o_x = 0, o_res = align256(H * 4), in_bytes = o_res + (residual ? H * 4 : 0);
  const size_t o_y = 0, o_ids = o_y + align256(H * 4), o_probs = o_ids + align256(K * 4),
               o_shg = o_probs + align256(K * 4), o_key = o_shg + 256,
               nkey = (size_t)(Ly->fused ? Ly->plan.grid : 1), bytes = o_key + nkey * 8;
  hipStream_t st = c->cur;
  HIP_TRY(c->pin.ensure(in_bytes));
  HIP_TRY(c->pin_out.ensure(bytes));
  uint8_t* hi = c->pin.p;
  uint8_t* di = c->pin.d;
  uint8_t* hb = c->pin_out.p;
  uint8_t* db = c->pin_out.d;
  memcpy(hi + o_x, x, H * 4);
  if (residual) memcpy(hi + o_res, residual, H * 4);
  const float* dx = reinterpret_cast<const float*>(di + o_x);
  const float* dres = residual ? reinterpret_cast<const float*>(di + o_res) : nullptr;
  float* dy = reinterpret_cast<float*>(db + o_y);
  int32_t* dids = reinterpret_cast<int32_t*>(db + o_ids);
  float* dprobs = reinterpret_cast<float*>(db + o_probs);
  float* dshg = reinterpret_cast<float*>(db + o_shg);
  if (!c->status_clean[layer]) HIP_TRY(reset_status(c, layer));
  size_t nk = 1;  // status words the last run left in the block
  volatile unsigned long long* keys = reinterpret_cast<unsigned long long*>(hb + o_key);
  auto run_and_fetch = [&](bool allow_fused) -> hipError_t {
    // The fused kernel's workgroups write the outputs and then the status
    // keys into the block themselves (fine-grained host memory), each key a
    // system-scope release after that workgroup's outputs, so once every key
    // word has changed from the sentinel the outputs are in place and the
    // call returns without the runtime's stream synchronisation (a poll of
    // the block instead).  A run that has not finished within kHostPollLimit
    // is left to hipStreamSynchronize, which also reports a failed launch.
    for (size_t i = 0; i < nkey; ++i) keys[i] = kKeySentinel;
    bool exported = false;
    hipError_t e = run_block(c, Ly, layer, dx, dres, 1, dy, dids, dprobs, dshg, allow_fused, nm,
                             nullptr, reinterpret_cast<unsigned long long*>(db + o_key), &exported);
    nk = exported ? nkey : 1;
    if (e != hipSuccess) return e;
    if (!exported) {
      e = hipMemcpyAsync(hb + o_key, c->status + layer, 8, hipMemcpyDeviceToHost, st);
      return e == hipSuccess ? hipStreamSynchronize(st) : e;
    }
    const auto t0 = std::chrono::steady_clock::now();
    for (size_t i = 0; i < nkey;) {
      if (keys[i] != kKeySentinel) {
        ++i;
        continue;
      }
      if (std::chrono::steady_clock::now() - t0 > kHostPollLimit) return hipStreamSynchronize(st);
    }
    std::atomic_thread_fence(std::memory_order_acquire);
    return hipSuccess;
  };
  auto key_of = [&]() {
    unsigned long long k = ~0ull, v;
    for (size_t i = 0; i < nk; ++i) {
      memcpy(&v, hb + o_key + i * 8, 8);
      k = v < k ? v : k;
    }
    return k;
  };
  HIP_TRY(run_and_fetch(true));
  c->last_ids[layer] = nullptr;  // the block is rewritten by the next call
  c->last_k[layer] = L.K;
  unsigned long long key = key_of();
  if (dm::key_phase(key) == dm::kPhExpert && dm::key_kind(key) == dm::kEkRecheck) {
    // see moe_forward_impl: the multi-kernel path names the failing check
    HIP_TRY(reset_status(c, layer));
    HIP_TRY(run_and_fetch(false));
    key = key_of();
  } else if (sync_timeout(key)) {
    // a wait of the persistent grid gave up (another process's kernels
    // held CUs it needed): start the tags again and rerun the token on the
    // multi-kernel path, which has no waits between workgroups
    HIP_TRY(hipStreamSynchronize(c->cur));
    HIP_TRY(reset_counters(c, Ly));
    HIP_TRY(reset_status(c, layer));
    HIP_TRY(run_and_fetch(false));
    key = key_of();
    ++c->sync_fallbacks;
  }
  memcpy(y, hb + o_y, H * 4);
  if (ids) memcpy(ids, hb + o_ids, K * 4);
  if (probs) memcpy(probs, hb + o_probs, K * 4);
  if (shg) memcpy(shg, hb + o_shg, 4);
  int rc = finish_status(c, Ly, layer, key, reinterpret_cast<const int32_t*>(hb + o_ids), err,
                         errlen);
  if (rc)
    HIP_TRY(reset_status(c, layer));
  else
    c->status_clean[layer] = 1;
  return rc;
}

// dmh_moe_forward and dmh_port_moe_forward: nm (may be NULL) normalises the
// block input first.
int moe_forward_impl(dmh_ctx* c, int layer, const float* x, const float* residual, int T,
                     float* y, int32_t* ids, float* probs, float* shg, unsigned flags,
                     const dm::NormSpec* nm, char* err, size_t errlen) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_moe_forward: layer %d not uploaded",
                   layer);
  if (!x || !y)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_moe_forward: x and y are required");
  if (T <= 0)
    return set_err(err, errlen, DMH_ERR_ACT,
                   "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"dimensions must be"
                   " positive\",\"stage\":\"router\",\"layer\":%d}", layer);
  HIP_TRY(hipSetDevice(c->device));
  const LayerDev& L = Ly->dev;
  const size_t TH = (size_t)T * L.H, TK = (size_t)T * L.K;
  const bool dev = flags & DMH_F_DEVICE;
  hipStream_t st = c->cur;
  if (dev) {
    int32_t* dids = ids;
    float* dprobs = probs;
    float* dshg = shg;
    if (!dids) { HIP_TRY(c->ids.ensure(TK)); dids = c->ids.p; }
    if (!dprobs) { HIP_TRY(c->probs.ensure(TK)); dprobs = c->probs.p; }
    if (!dshg) { HIP_TRY(c->shg.ensure(T)); dshg = c->shg.p; }
    HIP_TRY(run_block(c, Ly, layer, x, residual, T, y, dids, dprobs, dshg, true, nm));
    c->last_ids[layer] = dids;
    c->last_k[layer] = L.K;
    return DMH_OK;
  }
  if (T == 1) return moe_forward_host1(c, Ly, layer, x, residual, y, ids, probs, shg, nm, err,
                                       errlen);
  // Host pointers, several tokens: the inputs go through one page-locked
  // block and one copy, the outputs (with the status key) come back the
  // same way.
  const size_t in_bytes = align256(TH * 4) + (residual ? TH * 4 : 0);
  const size_t o_y = 0, o_ids = align256(o_y + TH * 4), o_probs = align256(o_ids + TK * 4),
               o_shg = align256(o_probs + TK * 4), o_key = align256(o_shg + (size_t)T * 4),
               out_bytes = o_key + 8;
  HIP_TRY(c->io_in.ensure(in_bytes));
  HIP_TRY(c->io_out.ensure(out_bytes));
  HIP_TRY(c->pin.ensure(align256(in_bytes) + out_bytes));
  uint8_t* hin = c->pin.p;
  uint8_t* hout = c->pin.p + align256(in_bytes);
  memcpy(hin, x, TH * 4);
  if (residual) memcpy(hin + align256(TH * 4), residual, TH * 4);
  uint8_t* din = c->io_in.p;
  uint8_t* dout = c->io_out.p;
  const float* dx = reinterpret_cast<const float*>(din);
  const float* dres = residual ? reinterpret_cast<const float*>(din + align256(TH * 4)) : nullptr;
  float* dy = reinterpret_cast<float*>(dout + o_y);
  int32_t* dids = reinterpret_cast<int32_t*>(dout + o_ids);
  float* dprobs = reinterpret_cast<float*>(dout + o_probs);
  float* dshg = reinterpret_cast<float*>(dout + o_shg);
  HIP_TRY(hipMemcpyAsync(din, hin, in_bytes, hipMemcpyHostToDevice, st));
  HIP_TRY(reset_status(c, layer));
  auto run_and_fetch = [&](bool allow_fused) -> hipError_t {
    hipError_t e = run_block(c, Ly, layer, dx, dres, T, dy, dids, dprobs, dshg, allow_fused, nm);
    if (e == hipSuccess)
      e = hipMemcpyAsync(dout + o_key, c->status + layer, 8, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(hout, dout, out_bytes, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e;
  };
  HIP_TRY(run_and_fetch(true));
  c->last_ids[layer] = dids;
  c->last_k[layer] = L.K;
  unsigned long long key;
  memcpy(&key, hout + o_key, 8);
  if (dm::key_phase(key) == dm::kPhExpert && dm::key_kind(key) == dm::kEkRecheck) {
    // The fused kernels fold the routed and shared down projections into one
    // sum, so a non-finite output does not say which check of the reference
    // fires first; the multi-kernel path keeps them apart and re-derives it.
    HIP_TRY(reset_status(c, layer));
    HIP_TRY(run_and_fetch(false));
    memcpy(&key, hout + o_key, 8);
  } else if (sync_timeout(key)) {
    // a wait of the several-token launch gave up: start the tags again and
    // rerun the tokens on the multi-kernel path (as the single-token call does)
    HIP_TRY(hipStreamSynchronize(st));
    HIP_TRY(reset_counters(c, Ly));
    HIP_TRY(reset_status(c, layer));
    HIP_TRY(run_and_fetch(false));
    memcpy(&key, hout + o_key, 8);
    ++c->sync_fallbacks;
  }
  memcpy(y, hout + o_y, TH * 4);
  if (ids) memcpy(ids, hout + o_ids, TK * 4);
  if (probs) memcpy(probs, hout + o_probs, TK * 4);
  if (shg) memcpy(shg, hout + o_shg, (size_t)T * 4);
  int rc = finish_status(c, Ly, layer, key, reinterpret_cast<const int32_t*>(hout + o_ids), err,
                         errlen);
  if (rc) HIP_TRY(reset_status(c, layer));
  return rc;
}

// rmsnorm's eps check (src/layers/rmsnorm.mojo:36-41).
int eps_check(float eps, char* err, size_t errlen) {
  if (!std::isfinite(eps) || eps <= 0.0f)
    return set_err(err, errlen, DMH_ERR_CONFIG,
                   "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"rms_norm_eps must be finite"
                   " and > 0\",\"stage\":\"config\"}");
  return DMH_OK;
}

}  // namespace

extern "C" {

int dmh_moe_forward(dmh_ctx* c, int layer, const float* x, const float* residual, int T,
                    float* y, int32_t* ids, float* probs, float* shg, unsigned flags, char* err,
                    size_t errlen) {
  return moe_forward_impl(c, layer, x, residual, T, y, ids, probs, shg, flags, nullptr, err,
                          errlen);
}

// dmh_moe_forward with every buffer of the call in this device's static
// scratch: no allocation of any kind.
int dmh_moe_forward_noalloc(dmh_ctx* c, int layer, const float* x, const float* residual, int T,
                            float* y, int32_t* ids, float* probs, float* shg, unsigned flags,
                            char* err, size_t errlen) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_moe_forward_noalloc: layer %d not uploaded", layer);
  if (!(flags & DMH_F_DEVICE))
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_moe_forward_noalloc: needs DMH_F_DEVICE (host pointers are staged "
                   "through allocated buffers)");
  if (!x || !y)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_moe_forward_noalloc: x and y are required");
  if (T <= 0)
    return set_err(err, errlen, DMH_ERR_ACT,
                   "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"dimensions must be"
                   " positive\",\"stage\":\"router\",\"layer\":%d}", layer);
  const LayerDev& L = Ly->dev;
  const size_t TK = (size_t)T * L.K;
  // scratch: the path's buffers, then ids / probs / shared gate when the
  // caller passes none
  const size_t need = scratch_carve(L, T, false, nullptr, nullptr) + (ids ? 0 : align256(TK * 4)) +
                      (probs ? 0 : align256(TK * 4)) + (shg ? 0 : align256((size_t)T * 4));
  if (need > kNoAllocScratchBytes)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_moe_forward_noalloc: seq_len %d needs %zu bytes of scratch, more than the"
                   " %zu bytes held per device", T, need, kNoAllocScratchBytes);
  HIP_TRY(hipSetDevice(c->device));
  uint8_t* base = (uint8_t*)g_scratch_dev[c->device];
  if (!base)
    return set_err(err, errlen, DMH_ERR_HIP, "dmh_moe_forward_noalloc: no scratch on device %d",
                   c->device);
  BlockScratch sc;
  size_t off = scratch_carve(L, T, false, base, &sc);
  if (!ids) { ids = (int32_t*)(base + off); off += align256(TK * 4); }
  if (!probs) { probs = (float*)(base + off); off += align256(TK * 4); }
  if (!shg) { shg = (float*)(base + off); off += align256((size_t)T * 4); }
  // One call at a time on this device's scratch: wait for the previous
  // call's kernels, whichever context queued them.  A stream being captured
  // cannot wait on an event recorded outside its capture; a captured call is
  // ordered only by the stream its graph is launched on.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(c->cur, &cap));
  const bool chain = cap == hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> order(g_scratch_mu);
  if (chain && g_noalloc_recorded[c->device])
    HIP_TRY(hipStreamWaitEvent(c->cur, g_noalloc_ev[c->device], 0));
  // the need-lo flag and the front-end counter start at zero (a call that
  // failed may have left the flag set)
  if (sc.needlo) HIP_TRY(dm::launch_fill_i32(sc.needlo, kFlagInts, 0, c->cur));
  HIP_TRY(run_block(c, Ly, layer, x, residual, T, y, ids, probs, shg, true, nullptr, &sc));
  if (chain) {
    HIP_TRY(hipEventRecord(g_noalloc_ev[c->device], c->cur));
    g_noalloc_recorded[c->device] = true;
  }
  c->last_ids[layer] = ids;
  c->last_k[layer] = L.K;
  return DMH_OK;
}

int dmh_port_moe_forward(dmh_ctx* c, int layer, const float* x_mid, int T, float eps, float* y,
                         int32_t* ids, float* probs, float* shg, unsigned flags, char* err,
                         size_t errlen) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_port_moe_forward: layer %d not uploaded",
                   layer);
  if (T <= 0)
    return set_err(err, errlen, DMH_ERR_NORM,
                   "{\"error_type\":\"NORM_ERROR\",\"detail\":\"empty input\",\"stage\":"
                   "\"rmsnorm\"}");
  int rc = eps_check(eps, err, errlen);
  if (rc) return rc;
  const dm::NormSpec nm = layer_norm(c, Ly, eps, (flags & DMH_F_NORM_TREE) != 0);
  return moe_forward_impl(c, layer, x_mid, x_mid, T, y, ids, probs, shg, flags, &nm, err, errlen);
}

int dmh_set_layer_norm(dmh_ctx* c, int layer, const float* gamma, int hidden, unsigned flags,
                       char* err, size_t errlen) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_set_layer_norm: layer %d not uploaded",
                   layer);
  if (hidden != Ly->dims.hidden)
    return set_err(err, errlen, DMH_ERR_NORM,
                   "{\"error_type\":\"NORM_ERROR\",\"detail\":\"length mismatch\",\"stage\":"
                   "\"rmsnorm\"}");
  HIP_TRY(hipSetDevice(c->device));
  HIP_TRY(hipStreamSynchronize(c->cur));
  if (!gamma) {
    if (Ly->gamma) HIP_TRY(hipFree(Ly->gamma));
    Ly->gamma = nullptr;
    return DMH_OK;
  }
  if (!Ly->gamma) HIP_TRY(hipMalloc(&Ly->gamma, sizeof(float) * (size_t)hidden));
  HIP_TRY(hipMemcpy(Ly->gamma, gamma, sizeof(float) * (size_t)hidden,
                    (flags & DMH_F_DEVICE) ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice));
  return DMH_OK;
}

int dmh_moe_stack_forward(dmh_ctx* c, int first, int nl, float eps, const float* x, int T,
                          float* out, int32_t* ids, float* probs, unsigned flags, char* err,
                          size_t errlen) {
  if (!c || !x || !out || nl <= 0 || T <= 0)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_moe_stack_forward: bad arguments");
  int rc0 = eps_check(eps, err, errlen);
  if (rc0) return rc0;
  Layer* L0 = get_layer(c, first);
  if (!L0)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_moe_stack_forward: layer %d missing",
                   first);
  const int H = L0->dims.hidden, K = L0->dims.top_k;
  for (int l = first; l < first + nl; ++l) {
    Layer* Ly = get_layer(c, l);
    if (!Ly || Ly->dims.hidden != H || Ly->dims.top_k != K)
      return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                     "dmh_moe_stack_forward: layer %d missing or of another shape", l);
  }
  HIP_TRY(hipSetDevice(c->device));
  const bool dev = flags & DMH_F_DEVICE;
  hipStream_t st = c->cur;
  const size_t TH = (size_t)T * H, TK = (size_t)T * K;
  HIP_TRY(c->hstack.ensure(2 * TH));
  float* hA = c->hstack.p;
  float* hB = c->hstack.p + TH;
  // device pointers: layer 0 reads x and the last layer writes out directly
  // (unless they alias); host pointers: x goes through hA
  const bool direct = dev && out != x;
  const bool own_ids = !(dev && ids), own_probs = !(dev && probs);
  if (own_ids) HIP_TRY(c->ids.ensure(TK * nl));
  if (own_probs) HIP_TRY(c->probs.ensure(TK * nl));
  HIP_TRY(c->shg.ensure(T));
  auto run_stack = [&](bool allow_fused) -> hipError_t {
    hipError_t e;
    const float* src = x;
    if (!direct) {
      if ((e = hipMemcpyAsync(hA, x, TH * 4,
                              dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st)) !=
          hipSuccess)
        return e;
      src = hA;
    }
    if (!dev)
      for (int l = first; l < first + nl; ++l)
        if ((e = reset_status(c, l)) != hipSuccess) return e;
    for (int i = 0; i < nl; ++i) {
      const int l = first + i;
      int32_t* dids = (own_ids ? c->ids.p : ids) + (size_t)i * TK;
      float* dprobs = (own_probs ? c->probs.p : probs) + (size_t)i * TK;
      float* dst = (direct && i == nl - 1) ? out : (src == hA ? hB : hA);
      const dm::NormSpec nm = layer_norm(c, c->layers[l], eps, (flags & DMH_F_NORM_TREE) != 0);
      if ((e = run_block(c, c->layers[l], l, src, src, T, dst, dids, dprobs, c->shg.p,
                         allow_fused, &nm)) != hipSuccess)
        return e;
      c->last_ids[l] = dids;
      c->last_k[l] = K;
      src = dst;
    }
    if (src != out &&
        (e = hipMemcpyAsync(out, src, TH * 4,
                            dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, st)) !=
            hipSuccess)
      return e;
    return hipSuccess;
  };
  HIP_TRY(run_stack(true));
  if (dev) return DMH_OK;
  std::vector<int32_t> hids(TK * nl);
  std::vector<unsigned long long> keys(nl);
  auto fetch = [&]() -> hipError_t {
    hipError_t e;
    if ((e = hipMemcpyAsync(hids.data(), c->ids.p, TK * nl * 4, hipMemcpyDeviceToHost, st)) !=
        hipSuccess)
      return e;
    if (probs && (e = hipMemcpyAsync(probs, c->probs.p, TK * nl * 4, hipMemcpyDeviceToHost,
                                     st)) != hipSuccess)
      return e;
    if ((e = hipMemcpyAsync(keys.data(), c->status + first, nl * 8, hipMemcpyDeviceToHost, st)) !=
        hipSuccess)
      return e;
    return hipStreamSynchronize(st);
  };
  HIP_TRY(fetch());
  bool timed_out = false;
  for (int i = 0; i < nl; ++i) timed_out |= sync_timeout(keys[i]);
  if (timed_out) {
    // a wait of a persistent grid gave up: start every layer's tags again and
    // rerun the stack on the multi-kernel path, which has no such waits
    for (int l = first; l < first + nl; ++l) HIP_TRY(reset_counters(c, c->layers[l]));
    HIP_TRY(run_stack(false));
    HIP_TRY(fetch());
    ++c->sync_fallbacks;
  }
  if (ids) memcpy(ids, hids.data(), TK * nl * 4);
  for (int i = 0; i < nl; ++i) {
    int rc = finish_status(c, c->layers[first + i], first + i, keys[i], hids.data() + i * TK, err,
                           errlen);
    if (rc) {
      for (int l = first; l < first + nl; ++l) HIP_TRY(reset_status(c, l));
      return rc;
    }
  }
  return DMH_OK;
}

int dmh_router_forward(dmh_ctx* c, const float* x, const float* w, int T, int H, int E, int K,
                       int norm, int layer, int32_t* ids, float* probs, unsigned flags, char* err,
                       size_t errlen) {
  if (!c || !x || !w || !ids || !probs)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_router_forward: NULL argument");
  int rc = router_config_check(E, K, norm, err, errlen);
  if (rc) return rc;
  if (T <= 0 || H <= 0)
    return set_err(err, errlen, DMH_ERR_ACT,
                   "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"dimensions must be"
                   " positive\",\"stage\":\"router\",\"layer\":%d}", layer);
  if (E > 2048)
    return set_err(err, errlen, DMH_ERR_CONFIG,
                   "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"num_experts > 2048 not"
                   " supported\",\"stage\":\"router\",\"layer\":%d}", layer);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->cur;
  const bool dev = flags & DMH_F_DEVICE;
  const size_t TH = (size_t)T * H, EH = (size_t)E * H, TK = (size_t)T * K;
  unsigned long long* status = c->status + kMaxLayers;
  const float *dx = x, *dw = w;
  int32_t* dids = ids;
  float* dprobs = probs;
  if (!dev) {
    HIP_TRY(c->x.ensure(TH));
    HIP_TRY(c->xn.ensure(EH));
    HIP_TRY(c->ids.ensure(TK));
    HIP_TRY(c->probs.ensure(TK));
    HIP_TRY(hipMemcpyAsync(c->x.p, x, TH * 4, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(c->xn.p, w, EH * 4, hipMemcpyHostToDevice, st));
    dx = c->x.p;
    dw = c->xn.p;
    dids = c->ids.p;
    dprobs = c->probs.p;
    HIP_TRY(reset_status(c, kMaxLayers));
  }
  HIP_TRY(c->z.ensure((size_t)T * E));
  HIP_TRY(dm::launch_router_generic(dx, dw, T, H, E, c->z.p, status, st));
  HIP_TRY(c->shg.ensure(T));
  HIP_TRY(dm::launch_router_select(c->z.p, E, T, E, K, 0, dids, dprobs, c->shg.p, status, st));
  if (dev) return DMH_OK;
  unsigned long long key = 0;
  HIP_TRY(hipMemcpyAsync(ids, dids, TK * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(probs, dprobs, TK * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(&key, status, 8, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (key == dm::kNoError) return DMH_OK;
  HIP_TRY(reset_status(c, kMaxLayers));
  return decode_key(key, layer, -1, E, err, errlen);
}

int dmh_dequant_q4_bf16(dmh_ctx* c, const uint16_t* scales, int64_t n_scales,
                        const uint8_t* packed, int64_t n_packed, int64_t n, int G, uint16_t* out,
                        unsigned flags, char* err, size_t errlen) {
  // validation order and messages of src/quant/dequant_kernel.mojo:33-66
  if (!(G == 32 || G == 64 || G == 128 || G == 256))
    return set_err(err, errlen, DMH_ERR_DEQUANT,
                   "dequant_kernel: group_size must be in {32, 64, 128, 256}, got %d", G);
  if (n <= 0)
    return set_err(err, errlen, DMH_ERR_DEQUANT, "dequant_kernel: num_elements must be positive");
  if (n % G != 0)
    return set_err(err, errlen, DMH_ERR_DEQUANT,
                   "M6_ERR_INPUT: N %% G != 0 (tail group not supported): N=%lld, G=%d",
                   (long long)n, G);
  if (n_scales != n / G)
    return set_err(err, errlen, DMH_ERR_DEQUANT,
                   "dequant_kernel: scales length mismatch: expected %lld, got %lld",
                   (long long)(n / G), (long long)n_scales);
  if (n_packed != (n + 1) / 2)
    return set_err(err, errlen, DMH_ERR_DEQUANT,
                   "dequant_kernel: packed weights length mismatch: expected %lld, got %lld",
                   (long long)((n + 1) / 2), (long long)n_packed);
  if (!c || !scales || !packed || !out)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_dequant_q4_bf16: NULL argument");
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->cur;
  const bool dev = flags & DMH_F_DEVICE;
  const uint16_t* ds = scales;
  const uint8_t* dp = packed;
  uint16_t* dout = out;
  if (!dev) {
    const size_t need = align256((size_t)n_scales * 2) + align256((size_t)n_packed) +
                        align256((size_t)n * 2);
    HIP_TRY(c->stage.ensure(need));
    uint8_t* b = c->stage.p;
    HIP_TRY(hipMemcpyAsync(b, scales, n_scales * 2, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(b + align256(n_scales * 2), packed, n_packed, hipMemcpyHostToDevice, st));
    ds = (const uint16_t*)b;
    dp = b + align256(n_scales * 2);
    dout = (uint16_t*)(b + align256(n_scales * 2) + align256(n_packed));
  }
  HIP_TRY(hipMemsetAsync(c->vkey, 0xFF, 8, st));
  HIP_TRY(dm::launch_dequant_ref(ds, dp, n, G, dout, c->vkey, st));
  unsigned long long vk = 0;
  HIP_TRY(hipMemcpyAsync(&vk, c->vkey, 8, hipMemcpyDeviceToHost, st));
  if (!dev) HIP_TRY(hipMemcpyAsync(out, dout, (size_t)n * 2, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (vk == dm::kNoError) return DMH_OK;
  if (vk == (1ull << 40))
    return set_err(err, errlen, DMH_ERR_DEQUANT,
                   "dequant_kernel: reserved nibble 0b1000 (-8) encountered");
  if (vk & 1ull)
    return set_err(err, errlen, DMH_ERR_DEQUANT, "dequant_kernel: scale is non-positive at group %llu",
                   (unsigned long long)(vk >> 1));
  return set_err(err, errlen, DMH_ERR_DEQUANT, "dequant_kernel: scale is NaN or Inf at group %llu",
                 (unsigned long long)(vk >> 1));
}

}  // extern "C"

// GGUF payload -> fp32 on the context's stream; raw and out each in host or
// device memory.  Shared by dmh_dequant_gguf and dmh_gguf_stream_tensor_f32.
int dm::api_dequant_gguf(dmh_ctx* c, int t, const void* raw, bool raw_dev, int64_t raw_bytes,
                         int64_t n, float* out, bool out_dev, int layout, char* err,
                         size_t errlen) {
  int bs = 0, bpb = 0;
  if (dm::gguf_block_spec(t, &bs, &bpb))
    return set_err(err, errlen, DMH_ERR_FORMAT, "GGUF_UNSUPPORTED_DTYPE: unsupported GGML type %d",
                   t);
  if (!c || !raw || !out || n < 0 || raw_bytes < 0)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_dequant_gguf: invalid argument");
  if (n == 0) return DMH_OK;
  const int64_t need = n / bs * bpb;
  if (raw_bytes < need)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_dequant_gguf: %lld payload bytes < %lld for %lld weights",
                   (long long)raw_bytes, (long long)need, (long long)n);
  if ((raw_dev && ((uintptr_t)raw & 3)) || (out_dev && ((uintptr_t)out & 15)))
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_dequant_gguf: device raw must be 4-byte and out 16-byte aligned");
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->cur;
  const size_t rb = raw_dev ? 0 : align256((size_t)(need > 0 ? need : 1));
  HIP_TRY(c->stage.ensure(rb + (out_dev ? 0 : (size_t)n * 4)));
  const uint8_t* draw = static_cast<const uint8_t*>(raw);
  float* dout = out;
  if (!raw_dev) {
    if (need > 0) HIP_TRY(hipMemcpyAsync(c->stage.p, raw, (size_t)need, hipMemcpyHostToDevice, st));
    draw = c->stage.p;
  }
  if (!out_dev) dout = reinterpret_cast<float*>(c->stage.p + rb);
  HIP_TRY(dm::launch_dequant_gguf(t, draw, n, layout, dout, st));
  if (!out_dev) HIP_TRY(hipMemcpyAsync(out, dout, (size_t)n * 4, hipMemcpyDeviceToHost, st));
  if (!(raw_dev && out_dev)) HIP_TRY(hipStreamSynchronize(st));
  return DMH_OK;
}

extern "C" {

int dmh_dequant_gguf(dmh_ctx* c, int t, const void* raw, int64_t raw_bytes, int64_t n, float* out,
                     unsigned flags, char* err, size_t errlen) {
  const bool dev = flags & DMH_F_DEVICE;
  return dm::api_dequant_gguf(c, t, raw, dev, raw_bytes, n, out, dev,
                              (flags & DMH_F_Q4K_PY_SCALES) ? 1 : 0, err, errlen);
}

int dmh_experts_forward(dmh_ctx* c, int layer, const float* x, int T, const int32_t* ids,
                        int K, float* out, float* shared_out, unsigned flags, char* err,
                        size_t errlen) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_experts_forward: layer %d not uploaded",
                   layer);
  if (!x || !ids || !out)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_experts_forward: x, ids and out are required");
  if (T <= 0 || K <= 0)
    return set_err(err, errlen, DMH_ERR_EXPERT,
                   "{\"error_type\":\"EXPERT_ERROR\",\"detail\":\"dimensions must be"
                   " positive\",\"stage\":\"swiglu\",\"layer\":%d}", layer);
  if (K > 64)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_experts_forward: top_k %d outside [1, 64]", K);
  HIP_TRY(hipSetDevice(c->device));
  const LayerDev& L = Ly->dev;
  const bool dev = flags & DMH_F_DEVICE;
  hipStream_t st = c->cur;
  unsigned long long* status = c->status + layer;
  c->status_clean[layer] = 0;
  const size_t TH = (size_t)T * L.H, TK = (size_t)T * K;
  std::vector<int32_t> hids;
  const float* dx = x;
  HIP_TRY(c->uids.ensure(TK));
  if (!dev) {
    hids.assign(ids, ids + TK);
    for (size_t i = 0; i < TK; ++i)
      if (hids[i] < 0 || hids[i] >= L.E)
        return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                       "{\"error_type\":\"EXPERT_ERROR\",\"detail\":\"expert id out of range\","
                       "\"stage\":\"swiglu\",\"layer\":%d,\"expert_id\":%d}", layer, hids[i]);
    HIP_TRY(c->x.ensure(TH));
    HIP_TRY(hipMemcpyAsync(c->x.p, x, TH * 4, hipMemcpyHostToDevice, st));
    dx = c->x.p;
    HIP_TRY(reset_status(c, layer));
    HIP_TRY(hipMemcpyAsync(c->uids.p, hids.data(), TK * 4, hipMemcpyHostToDevice, st));
  } else {
    HIP_TRY(dm::launch_check_ids(ids, T, K, L.E, c->uids.p, status, st));
  }
  // the grouped experts with K assignments per token
  LayerDev Lk = L;
  Lk.K = K;
  HIP_TRY(c->g_off.ensure(L.E + 1));
  HIP_TRY(c->g_perm.ensure(TK));
  HIP_TRY(c->g_meta.ensure(2));
  HIP_TRY(c->g_needlo.ensure(1));
  HIP_TRY(c->g_units.ensure(dm::group_units_max(T, K, L.E)));
  HIP_TRY(c->g_xhi.ensure(TH));
  HIP_TRY(c->g_xlo.ensure(TH));
  HIP_TRY(c->g_hr.ensure(2 * TK * L.I));
  HIP_TRY(c->g_hs.ensure(2 * (size_t)T * L.Ish));
  float* dout = dev ? out : nullptr;
  if (!dout) { HIP_TRY(c->g_r.ensure(TK * L.H)); dout = c->g_r.p; }
  HIP_TRY(c->g_rs.ensure(TH));
  HIP_TRY(hipMemsetAsync(c->g_needlo.p, 0, sizeof(int), st));
  HIP_TRY(dm::launch_split_rows(dx, (int64_t)TH, c->g_xhi.p, c->g_xlo.p, c->g_needlo.p, st));
  HIP_TRY(dm::launch_group_build(c->uids.p, T, K, L.E, c->g_off.p, c->g_perm.p, c->g_units.p,
                                 c->g_meta.p, st));
  float* drs = (dev && shared_out) ? shared_out : c->g_rs.p;
  HIP_TRY(dm::launch_experts_grouped(Lk, c->g_xhi.p, c->g_xlo.p, c->g_needlo.p, c->g_off.p,
                                     c->g_perm.p, c->g_units.p, c->g_meta.p, T, c->g_hr.p,
                                     c->g_hr.p + TK * L.I, c->g_hs.p,
                                     c->g_hs.p + (size_t)T * L.Ish, dout, drs, status, st));
  // leave the need-lo flag zero, as the block forward expects between calls
  HIP_TRY(hipMemsetAsync(c->g_needlo.p, 0, sizeof(int), st));
  c->last_ids[layer] = c->uids.p;
  c->last_k[layer] = K;
  if (dev) return DMH_OK;
  unsigned long long key = 0;
  HIP_TRY(hipMemcpyAsync(out, dout, TK * L.H * 4, hipMemcpyDeviceToHost, st));
  if (shared_out) HIP_TRY(hipMemcpyAsync(shared_out, drs, TH * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(&key, status, sizeof(key), hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  int rc = finish_status(c, Ly, layer, key, hids.data(), err, errlen, K);
  if (rc) HIP_TRY(reset_status(c, layer));
  return rc;
}

int dmh_shared_gate_forward(dmh_ctx* c, int layer, const float* x, int T, float* scores,
                            unsigned flags, char* err, size_t errlen) {
  Layer* Ly = get_layer(c, layer);
  if (!Ly)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_shared_gate_forward: layer %d not uploaded", layer);
  if (!x || !scores)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_shared_gate_forward: x and scores are required");
  if (T <= 0)
    return set_err(err, errlen, DMH_ERR_GATE,
                   "{\"error_type\":\"GATE_ERROR\",\"detail\":\"dimensions must be"
                   " positive\",\"stage\":\"shared\",\"layer\":%d}", layer);
  HIP_TRY(hipSetDevice(c->device));
  const LayerDev& L = Ly->dev;
  const bool dev = flags & DMH_F_DEVICE;
  hipStream_t st = c->cur;
  unsigned long long* status = c->status + layer;
  c->status_clean[layer] = 0;
  const size_t TH = (size_t)T * L.H;
  const float* dx = x;
  float* ds = dev ? scores : nullptr;
  if (!dev) {
    HIP_TRY(c->x.ensure(TH));
    HIP_TRY(hipMemcpyAsync(c->x.p, x, TH * 4, hipMemcpyHostToDevice, st));
    dx = c->x.p;
    HIP_TRY(c->shg.ensure(T));
    ds = c->shg.p;
    HIP_TRY(reset_status(c, layer));
  }
  // the gate vector is row E of the router layout: the lane-chain router on
  // that one row gives the logit in the order of shared_gate_forward
  // (src/layers/moe.mojo:64-81); the activation scan of that kernel goes to
  // a scratch word, as shared_gate_forward has none
  LayerDev Lg = L;
  Lg.router = L.router + (size_t)L.E * L.H;
  Lg.E = 0;
  HIP_TRY(c->z.ensure(T));
  HIP_TRY(dm::launch_router_dec(Lg, dx, T, c->z.p, c->vkey, st));
  HIP_TRY(dm::launch_shared_gate_scores(c->z.p, 1, T, ds, status, st));
  if (dev) return DMH_OK;
  unsigned long long key = 0;
  HIP_TRY(hipMemcpyAsync(scores, ds, (size_t)T * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(&key, status, sizeof(key), hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  int rc = finish_status(c, Ly, layer, key, nullptr, err, errlen);
  if (rc) HIP_TRY(reset_status(c, layer));
  return rc;
}

int dmh_moe_aggregate(dmh_ctx* c, const float* residual, const float* routed, const float* probs,
                      const float* shared_out, const float* shared_gates, int T, int H, int K,
                      int layer, float* out, unsigned flags, char* err, size_t errlen) {
  if (!c || !routed || !probs || !shared_out || !shared_gates || !out)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_moe_aggregate: NULL argument");
  if (T <= 0 || H <= 0 || K < 0)
    return set_err(err, errlen, DMH_ERR_EXPERT,
                   "{\"error_type\":\"EXPERT_ERROR\",\"detail\":\"dimensions must be"
                   " positive\",\"stage\":\"aggregation\",\"layer\":%d}", layer);
  HIP_TRY(hipSetDevice(c->device));
  const bool dev = flags & DMH_F_DEVICE;
  hipStream_t st = c->cur;
  unsigned long long* status = c->status + kMaxLayers;
  const size_t TH = (size_t)T * H, TK = (size_t)T * K;
  const float *dr = routed, *dp = probs, *dsh = shared_out, *dg = shared_gates, *dres = residual;
  float* dy = out;
  if (!dev) {
    HIP_TRY(c->g_r.ensure(TK * H > 0 ? TK * H : 1));
    HIP_TRY(c->g_rs.ensure(TH));
    HIP_TRY(c->probs.ensure(TK > 0 ? TK : 1));
    HIP_TRY(c->shg.ensure(T));
    HIP_TRY(c->y.ensure(TH));
    if (TK) HIP_TRY(hipMemcpyAsync(c->g_r.p, routed, TK * H * 4, hipMemcpyHostToDevice, st));
    if (TK) HIP_TRY(hipMemcpyAsync(c->probs.p, probs, TK * 4, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(c->g_rs.p, shared_out, TH * 4, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(c->shg.p, shared_gates, (size_t)T * 4, hipMemcpyHostToDevice, st));
    dr = c->g_r.p;
    dp = c->probs.p;
    dsh = c->g_rs.p;
    dg = c->shg.p;
    dy = c->y.p;
    if (residual) {
      HIP_TRY(c->res.ensure(TH));
      HIP_TRY(hipMemcpyAsync(c->res.p, residual, TH * 4, hipMemcpyHostToDevice, st));
      dres = c->res.p;
    }
    HIP_TRY(reset_status(c, kMaxLayers));
  }
  HIP_TRY(dm::launch_combine(dr, dsh, dp, dg, dres, T, H, K, dy, status, st));
  if (dev) return DMH_OK;
  unsigned long long key = 0;
  HIP_TRY(hipMemcpyAsync(out, dy, TH * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(&key, status, sizeof(key), hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (key == dm::kNoError) return DMH_OK;
  HIP_TRY(reset_status(c, kMaxLayers));
  return decode_key(key, layer, -1, 0, err, errlen);
}

// load_port_block_from_gguf's MoE tensors (src/layers/gguf_port_loader.mojo:
// 207-256) -> one GGUF layer in HBM.  Lookup, read, type and length checks
// run in the loader's order with its texts.
static int upload_gguf_body(dmh_ctx* c, int layer, const dmh_moe_dims* d,
                            const dmh_gguf_file* gf, int model_layer, unsigned flags, char* err,
                            size_t errlen);

// Host vectors grow with the file's payload: nothing may throw across the ABI.
int dmh_upload_moe_layer_gguf(dmh_ctx* c, int layer, const dmh_moe_dims* d,
                              const dmh_gguf_file* gf, int model_layer, unsigned flags, char* err,
                              size_t errlen) {
  try {
    return upload_gguf_body(c, layer, d, gf, model_layer, flags, err, errlen);
  } catch (const std::bad_alloc&) {
    return set_err(err, errlen, DMH_ERR_NO_MEMORY, "dmh_upload_moe_layer_gguf: out of host memory");
  } catch (const std::exception& ex) {
    return set_err(err, errlen, DMH_ERR_NO_MEMORY, "dmh_upload_moe_layer_gguf: %s", ex.what());
  }
}

static int upload_gguf_body(dmh_ctx* c, int layer, const dmh_moe_dims* d,
                            const dmh_gguf_file* gf, int model_layer, unsigned flags, char* err,
                            size_t errlen) {
  if (!c || !d || !gf)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_upload_moe_layer_gguf: NULL argument");
  if (layer < 0 || layer >= kMaxLayers)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_upload_moe_layer_gguf: layer %d outside [0, %d)", layer, kMaxLayers);
  const int H = d->hidden, E = d->num_experts, K = d->top_k, I = d->inter, Ish = d->inter_sh;
  int rc = router_config_check(E, K, d->norm_topk_prob, err, errlen);
  if (rc) return rc;
  if (H <= 0 || I <= 0 || Ish <= 0 || H % 4 || I % 4 || Ish % 4 || E > 2048 || K > 32)
    return set_err(err, errlen, DMH_ERR_CONFIG,
                   "{\"error_type\":\"CONFIG_ERROR\",\"detail\":\"GGUF layer needs hidden, inter"
                   " and shared inter positive multiples of 4, num_experts <= 2048, top_k <= 32\""
                   ",\"stage\":\"loader\",\"layer\":%d}", layer);
  const dm::GgufFile& f = gf->f;
  const std::string pfx = "blk." + std::to_string(model_layer) + ".";
  // payload of one tensor, with the checks of stream_gguf_tensor_f32 and
  // _expect_len (gguf_port_loader.mojo:55-67)
  auto load = [&](const std::string& name, int64_t want, std::vector<uint8_t>* raw,
                  int* type) -> int {
    const int idx = f.find(name);
    if (idx < 0)
      return set_err(err, errlen, DMH_ERR_WEIGHT,
                     "{\"error_type\":\"WEIGHT_LOAD_FAILED\",\"detail\":\"tensor not found in GGUF"
                     " index\",\"tensor\":\"%s\"}", name.c_str());
    std::string e;
    if (!dm::read_gguf_tensor(f, idx, raw, &e)) return set_err(err, errlen, DMH_ERR_WEIGHT, "%s", e.c_str());
    const dm::GgufTensor& t = f.tensors[idx];
    int bs, bpb;
    if (dm::gguf_block_spec(t.type, &bs, &bpb))
      return set_err(err, errlen, DMH_ERR_FORMAT,
                     "GGUF_UNSUPPORTED_DTYPE: unsupported GGML type %d for tensor %s", t.type,
                     name.c_str());
    if (t.num_elements != want)
      return set_err(err, errlen, DMH_ERR_FORMAT,
                     "GGUF_FILE_CORRUPT: dimension mismatch for tensor %s: expected %lld elements,"
                     " got %lld", name.c_str(), (long long)want, (long long)t.num_elements);
    *type = t.type;
    return DMH_OK;
  };
  std::vector<uint8_t> router_raw, sg_raw, tmp;
  int router_t = 0, sg_t = 0, exp_t = -1, ty = 0;
  if ((rc = load(pfx + "ffn_gate_exps.weight", (int64_t)E * H, &router_raw, &router_t))) return rc;
  // expert payloads back to back, each 256-byte aligned; row E = shared
  std::vector<int64_t> off((size_t)(E + 1) * 3);
  std::vector<uint8_t> payload;
  auto append = [&](const std::string& name, int64_t want, int64_t* o) -> int {
    int r = load(name, want, &tmp, &ty);
    if (r) return r;
    if (exp_t >= 0 && ty != exp_t)
      return set_err(err, errlen, DMH_ERR_FORMAT,
                     "dmh_upload_moe_layer_gguf: expert tensor %s has GGML type %d, the others %d",
                     name.c_str(), ty, exp_t);
    // the reference leaves the weights of a partial last block at 0.0; the
    // expert kernels decode whole blocks only
    int bs = 1, bpb = 0;
    dm::gguf_block_spec(ty, &bs, &bpb);
    if (want % bs)
      return set_err(err, errlen, DMH_ERR_FORMAT,
                     "dmh_upload_moe_layer_gguf: expert tensor %s has %lld weights, not whole "
                     "blocks of %d", name.c_str(), (long long)want, bs);
    exp_t = ty;
    *o = (int64_t)payload.size();
    payload.insert(payload.end(), tmp.begin(), tmp.end());
    payload.resize(align256(payload.size()), 0);
    return DMH_OK;
  };
  const int64_t IH = (int64_t)I * H, ShH = (int64_t)Ish * H;
  for (int e = 0; e < E; ++e) {
    const std::string es = std::to_string(e);
    if ((rc = append(pfx + "ffn_gate." + es + ".weight", IH, &off[(size_t)e * 3 + 0]))) return rc;
    if ((rc = append(pfx + "ffn_up." + es + ".weight", IH, &off[(size_t)e * 3 + 1]))) return rc;
    if ((rc = append(pfx + "ffn_down." + es + ".weight", IH, &off[(size_t)e * 3 + 2]))) return rc;
  }
  if ((rc = append(pfx + "ffn_shared_gate.weight", ShH, &off[(size_t)E * 3 + 0]))) return rc;
  if ((rc = append(pfx + "ffn_shared_up.weight", ShH, &off[(size_t)E * 3 + 1]))) return rc;
  if ((rc = append(pfx + "ffn_shared_down.weight", ShH, &off[(size_t)E * 3 + 2]))) return rc;
  if ((rc = load(pfx + "shared_gate.weight", H, &sg_raw, &sg_t))) return rc;

  HIP_TRY(hipSetDevice(c->device));
  hipStream_t st = c->cur;
  const size_t b_router = align256((size_t)E * H * 4), b_sg = align256((size_t)H * 4),
               b_off = align256(off.size() * 8), b_rr = align256(router_raw.size()),
               b_sr = align256(sg_raw.size());
  const size_t bytes = b_router + b_sg + b_off + payload.size() + b_rr + b_sr;
  GgufLayer* G = new GgufLayer();
  if (hipMalloc(&G->buf, bytes) != hipSuccess) {
    delete G;
    return set_err(err, errlen, DMH_ERR_NO_MEMORY,
                   "dmh_upload_moe_layer_gguf: cannot allocate %zu bytes", bytes);
  }
  uint8_t* b = static_cast<uint8_t*>(G->buf);
  float* d_router = reinterpret_cast<float*>(b);
  float* d_sg = reinterpret_cast<float*>(b + b_router);
  int64_t* d_off = reinterpret_cast<int64_t*>(b + b_router + b_sg);
  uint8_t* d_raw = b + b_router + b_sg + b_off;
  // the raw router and gate sit at the end of the block until dequantized
  uint8_t* d_rr = d_raw + payload.size();
  uint8_t* d_sr = d_rr + b_rr;
  const int layout = (flags & DMH_F_Q4K_PY_SCALES) ? 1 : 0;
  hipError_t e = hipMemcpyAsync(d_off, off.data(), off.size() * 8, hipMemcpyHostToDevice, st);
  if (e == hipSuccess && !payload.empty())
    e = hipMemcpyAsync(d_raw, payload.data(), payload.size(), hipMemcpyHostToDevice, st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d_rr, router_raw.data(), router_raw.size(), hipMemcpyHostToDevice, st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d_sr, sg_raw.data(), sg_raw.size(), hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = dm::launch_dequant_gguf(router_t, d_rr, (int64_t)E * H, layout, d_router, st);
  if (e == hipSuccess) e = dm::launch_dequant_gguf(sg_t, d_sr, H, layout, d_sg, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    (void)hipFree(G->buf);
    delete G;
    HIP_TRY(e);
  }
  G->dims = *d;
  G->bytes = bytes;
  // routed expert tensors of one size, appended in order from offset 0:
  // their offsets are (3e + k) * stride, no table lookup needed
  int64_t estride = off.size() > 1 ? off[1] - off[0] : 0;
  for (int i = 0; i < 3 * E && estride > 0; ++i)
    if (off[i] != (int64_t)i * estride) estride = 0;
  G->dev = dm::GgufMoeDev{H, E, K, I, Ish, exp_t, layout, d_raw, d_off, d_router, d_sg, estride};
  // the single-token form when its launch fits the device at once
  {
    int per_cu = 0;
    G->sync_bytes = dm::gguf_one_token_sync_bytes(G->dev);
    if (dm::gguf_one_token_supported(G->dev) && dm::gguf_one_token_grid_ok(G->dev, c->num_cus) &&
        dm::gguf_experts_occupancy(G->dev, &per_cu) == 0 && per_cu >= 1 &&
        hipMalloc(&G->sync, G->sync_bytes) == hipSuccess) {
      if (hipMalloc(&G->rchain, dm::gguf_chain_router_bytes(G->dev)) == hipSuccess &&
          dm::launch_chain_router(G->dev, G->rchain, st) == hipSuccess &&
          hipMemsetAsync(G->sync, 0, G->sync_bytes, st) == hipSuccess &&
          hipStreamSynchronize(st) == hipSuccess) {
        G->dev.rchain = G->rchain;
        G->grid = c->num_cus;
      } else {
        (void)hipFree(G->sync);
        G->sync = nullptr;
        if (G->rchain) (void)hipFree(G->rchain);
        G->rchain = nullptr;
      }
    }
  }
  if (GgufLayer* old = c->glayers[layer]) {
    (void)hipStreamSynchronize(st);
    free_glayer(old);
  }
  c->glayers[layer] = G;
  HIP_TRY(reset_status(c, kGgufSlot0 + layer));
  return DMH_OK;
}

int dmh_free_layer_gguf(dmh_ctx* c, int layer) {
  GgufLayer* G = get_glayer(c, layer);
  if (!G) return DMH_ERR_INVALID_ARG;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->cur);
  free_glayer(G);
  c->glayers[layer] = nullptr;
  return DMH_OK;
}

int dmh_moe_forward_gguf(dmh_ctx* c, int layer, const float* x, const float* residual, int T,
                         float* y, int32_t* ids, float* probs, float* shg, unsigned flags,
                         char* err, size_t errlen) {
  GgufLayer* G = get_glayer(c, layer);
  if (!G)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_moe_forward_gguf: GGUF layer %d not uploaded", layer);
  if (!x || !y)
    return set_err(err, errlen, DMH_ERR_INVALID_ARG, "dmh_moe_forward_gguf: x and y are required");
  if (T <= 0)
    return set_err(err, errlen, DMH_ERR_ACT,
                   "{\"error_type\":\"ACT_LOAD_FAILED\",\"detail\":\"dimensions must be"
                   " positive\",\"stage\":\"router\",\"layer\":%d}", layer);
  const bool dev = flags & DMH_F_DEVICE;
  if (dev && (((uintptr_t)x & 15) || ((uintptr_t)y & 15) || ((uintptr_t)residual & 15)))
    return set_err(err, errlen, DMH_ERR_INVALID_ARG,
                   "dmh_moe_forward_gguf: device x, residual and y must be 16-byte aligned");
  HIP_TRY(hipSetDevice(c->device));
  const dm::GgufMoeDev& L = G->dev;
  const size_t TH = (size_t)T * L.H, TK = (size_t)T * L.K;
  hipStream_t st = c->cur;
  unsigned long long* status = c->status + kGgufSlot0 + layer;
  if (dev) {
    int32_t* dids = ids;
    float* dprobs = probs;
    float* dshg = shg;
    if (!dids) { HIP_TRY(c->ids.ensure(TK)); dids = c->ids.p; }
    if (!dprobs) { HIP_TRY(c->probs.ensure(TK)); dprobs = c->probs.p; }
    if (!dshg) { HIP_TRY(c->shg.ensure(T)); dshg = c->shg.p; }
    HIP_TRY(run_gguf_block(c, G, status, x, residual, T, y, dids, dprobs, dshg));
    return DMH_OK;
  }
  HIP_TRY(c->x.ensure(TH));
  HIP_TRY(c->y.ensure(TH));
  HIP_TRY(c->ids.ensure(TK));
  HIP_TRY(c->probs.ensure(TK));
  HIP_TRY(c->shg.ensure(T));
  HIP_TRY(hipMemcpyAsync(c->x.p, x, TH * 4, hipMemcpyHostToDevice, st));
  const float* dres = nullptr;
  if (residual) {
    HIP_TRY(c->res.ensure(TH));
    HIP_TRY(hipMemcpyAsync(c->res.p, residual, TH * 4, hipMemcpyHostToDevice, st));
    dres = c->res.p;
  }
  HIP_TRY(reset_status(c, kGgufSlot0 + layer));
  HIP_TRY(run_gguf_block(c, G, status, c->x.p, dres, T, c->y.p, c->ids.p, c->probs.p, c->shg.p));
  unsigned long long key = 0;
  HIP_TRY(hipMemcpyAsync(&key, status, 8, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (sync_timeout(key)) {
    // a wait of the single-token grid gave up: start its tags again and
    // rerun the token on the four-launch path, which has no such waits
    if (G->sync) {
      HIP_TRY(hipMemsetAsync(G->sync, 0, G->sync_bytes, st));
      G->launches = 0;
    }
    HIP_TRY(reset_status(c, kGgufSlot0 + layer));
    HIP_TRY(run_gguf_block(c, G, status, c->x.p, dres, T, c->y.p, c->ids.p, c->probs.p, c->shg.p,
                           false));
    ++c->sync_fallbacks;
  }
  HIP_TRY(hipMemcpyAsync(y, c->y.p, TH * 4, hipMemcpyDeviceToHost, st));
  if (ids) HIP_TRY(hipMemcpyAsync(ids, c->ids.p, TK * 4, hipMemcpyDeviceToHost, st));
  if (probs) HIP_TRY(hipMemcpyAsync(probs, c->probs.p, TK * 4, hipMemcpyDeviceToHost, st));
  if (shg) HIP_TRY(hipMemcpyAsync(shg, c->shg.p, (size_t)T * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(&key, status, 8, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  if (key == dm::kNoError) return DMH_OK;
  HIP_TRY(reset_status(c, kGgufSlot0 + layer));
  return gguf_finish(c, layer, key, err, errlen);
}

}  // extern "C"
