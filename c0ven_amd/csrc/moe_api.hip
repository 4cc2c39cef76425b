// The C ABI (include/c0ven_moe.h): contexts, resident weights in the device layout, and the forward calls.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstddef>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/c0ven_moe.h"
#include "aux.h"
#include "decode.h"
#include "gguf_index.h"
#include "iq3s_grid.h"
#include "layout.h"
#include "prefill.h"
#include "prefill_hc.h"
#include "repack.h"

using namespace c0ven;

namespace {

struct Error : std::runtime_error {
  moe_status st;
  Error(moe_status s, const std::string &m) : std::runtime_error(m), st(s) {}
};

void check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw Error(MOE_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}
void require(bool ok, const std::string &why) {
  if (!ok) throw Error(MOE_BAD_ARGUMENT, why);
}

bool pow2(uint32_t v) { return v && !(v & (v - 1)); }

struct Layer {
  uint16_t *router = nullptr;
  uint16_t *router_t = nullptr;  // the routed rows in 16 x 32 tiles (the prefill router's operand)
  float *bias = nullptr;
  bool has_bias = false;
  float rmax = 0.0f, bias_max = 0.0f;  // the largest routed row norm and |bias| (the prefill router's bound)
  int *rlsb = nullptr;                 // per routed row: the least lsb of its bf16 values (its exact-sum condition)
  uint8_t *resident = nullptr;         // n_expert flags: the experts on the device (when has_miss)
  bool has_miss = false;               // some routed expert is not on the device
  uint8_t *experts = nullptr;
  uint8_t *shared = nullptr;
  // The hyper-connection module before the block (hc_lr > 0).
  float *hc_gamma = nullptr;
  uint16_t *hc_down = nullptr, *hc_inj = nullptr, *hc_up = nullptr;
  double *hc_rn = nullptr;  // the 2-norms of W_down's, W_inject's and W_up's rows (the prefill mix's bound)
  int *hc_rlsb = nullptr;   // the least lsb exponent of each of those rows' nonzero bf16 values
  bool has_hc = false;
};

constexpr uint32_t kMaxPrefillTokens = 16384;  // tokens one forward takes (one prefill chunk)

// A kernel launch timed with two events on its stream.
struct TimedLaunch {
  const char *name;
  hipEvent_t a, b;
};

// A kernel's timed launches folded into a sum (the event pool is bounded: past kTimedFold pending launches the record
// waits for them and folds them here).
struct TimedSum {
  const char *name;
  double ms;
  uint32_t n;
};
constexpr size_t kTimedFold = 4096;

// Device memory released when the scope ends, also when a check throws.
struct DevBuf {
  void *p = nullptr;
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
};

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// The decode kernel's scratch for moe_forward_async_noalloc: one array per GPU, in the library's own device memory
// (no call allocates it). Host code never passes the array's name to a kernel: on the host that name is a stand-in,
// not a device address. Each device's address comes from hipGetSymbolAddress, taken once per device (with it
// current) when the first context opens on it, and is used everywhere instead. Calls on one GPU share the array and
// the launch tags below, so they must be ordered (one stream, or event waits); overlapping calls race.
constexpr uint64_t kNoAllocScratchBytes = 16ull << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

struct NoAllocScratch {
  uint8_t *ptr = nullptr;            // this device's copy of `scratch`
  std::atomic<uint64_t> epoch{0};    // the last no-alloc launch's number on this device (tags every record)
};
NoAllocScratch g_noalloc[kMaxDevices];
std::mutex g_noalloc_mu;

// Zeroes n words (a fill kernel, not hipMemsetAsync: the no-alloc path may be captured into a HIP graph).
__global__ void fill_zero_u32(uint32_t *p, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

void zero_words(void *p, uint64_t bytes, hipStream_t s) {
  const uint64_t n = bytes / 4;
  hipLaunchKernelGGL(fill_zero_u32, dim3((uint32_t)std::min<uint64_t>((n + 255) / 256, 2048)), dim3(256), 0, s,
                     (uint32_t *)p, n);
  check(hipGetLastError(), "fill_zero_u32");
}

// Once per device (the device current): the array's address, and its contents zeroed (tag 0 is never a launch's).
void noalloc_setup(int dev) {
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  NoAllocScratch &d = g_noalloc[dev];
  if (d.ptr) return;
  void *ptr = nullptr;
  check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  zero_words(ptr, kNoAllocScratchBytes, nullptr);
  check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  d.ptr = (uint8_t *)ptr;
}

// Where the decode scratch of a context's shape sits inside a base (the array's device address, or null to size it).
struct NoAllocLayout {
  uint8_t *act_r, *act_s;
  uint64_t *logits, *gs, *ids_t, *w_t, *h, *y_asg, *flags;
  int32_t *ids;
  float *w;
  MoeGroup *groups;
  uint32_t *ngroups, *counters;
  uint64_t bytes, tagged_bytes;  // all of it; the leading part of it that holds tagged records and counters
};

NoAllocLayout noalloc_layout(const moe_config &g, uint8_t *base) {
  const uint32_t T = std::min<uint32_t>(g.max_tokens, kMaxDecodeTokens), K1 = g.n_used + 1;
  const uint32_t A = T * K1 + T, Ug = units_of(g.n_embd), E = g.n_expert;
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) {
    uint8_t *q = base ? base + off : nullptr;
    off += (bytes + 255) / 256 * 256;
    return q;
  };
  NoAllocLayout L{};
  // The counters and flags first, at the same place for every shape: contexts of different shapes share them, and a
  // launch relies on the previous launch (of any context) having reset the list counters it will use. Then the
  // tagged records: with the counters and flags, the part a tag wrap clears.
  L.counters = (uint32_t *)take((uint64_t)(3 + 2 * kDynLists * kDynStride + kDynStride) * 4);
  L.flags = (uint64_t *)take((uint64_t)kFlagCount * 8);
  L.logits = (uint64_t *)take((uint64_t)T * (E + 1) * 8);
  L.gs = (uint64_t *)take((uint64_t)T * 8);
  L.ids_t = (uint64_t *)take((uint64_t)T * K1 * 8);
  L.w_t = (uint64_t *)take((uint64_t)T * K1 * 8);
  L.h = (uint64_t *)take((uint64_t)A * g.n_ff * 8);
  L.y_asg = (uint64_t *)take((uint64_t)A * g.n_embd * 8);
  L.tagged_bytes = off;
  L.act_r = take((uint64_t)T * Ug * kActBytes);
  L.act_s = take((uint64_t)T * Ug * kActBytes);
  L.ids = (int32_t *)take((uint64_t)T * K1 * 4);
  L.w = (float *)take((uint64_t)T * K1 * 4);
  L.groups = (MoeGroup *)take((uint64_t)max_groups(T, K1) * sizeof(MoeGroup));
  L.ngroups = (uint32_t *)take(4);
  L.bytes = off;
  return L;
}

}  // namespace

struct moe_ctx {
  moe_config cfg{};
  hipStream_t stream = nullptr;
  std::vector<Layer> layers;
  uint64_t ex_bytes = 0, ex_up = 0, ex_down = 0, sh_bytes = 0, sh_up = 0, sh_down = 0;
  uint32_t tmax = 0, tdec = 0, k1 = 0, gmax = 0;  // tokens a forward takes; of them, the decode kernel's
  PfBufs pf{};                                      // prefill scratch (max_tokens > tdec)
  const int32_t *last_ids = nullptr;                // where the last forward left its ids and weights
  const float *last_w = nullptr;
  uint32_t last_pf_T = 0;                           // tokens of the last prefill forward
  // Staging for the host-memory calls.
  float *x_dev = nullptr, *y_dev = nullptr, *w_stage = nullptr;
  int32_t *ids_stage = nullptr;
  // Scratch.
  uint8_t *act_r = nullptr, *act_s = nullptr;
  float *w = nullptr;
  uint64_t *y_asg = nullptr, *logits = nullptr, *gs = nullptr, *h = nullptr, *ids_t = nullptr, *w_t = nullptr;  // tagged records
  int32_t *ids = nullptr;
  MoeGroup *groups = nullptr;
  uint32_t *ngroups = nullptr, *counters = nullptr, *tok_need = nullptr;
  uint32_t *cnt_route = nullptr, *cnt_topk = nullptr, *cnt_dyn = nullptr;
  uint32_t *err_flag = nullptr;
  uint64_t *flags = nullptr;
  uint64_t noalloc_bytes = 0;  // the no-alloc path's share of the device's scratch array for this shape
  // The hybrid's records and answer in pinned host memory (moe_miss_buffers), and their device addresses.
  uint8_t *miss_host = nullptr, *miss_dev = nullptr;
  uint64_t miss_stride = 0;
  uint32_t last_step = 0;
  // moe_compute_many's device copies of borrowed experts (routed types, ex_bytes each), keyed by gate pointer.
  uint8_t *bc_base = nullptr;
  uint32_t bc_slots = 0;
  std::vector<const uint8_t *> bc_key;
  std::vector<uint64_t> bc_used;  // the call that last used the slot
  uint64_t bc_calls = 0;
  uint64_t epoch = 0;          // the last launch's number
  std::vector<std::pair<uint64_t *, uint64_t>> tagged;  // the tagged-record buffers (pointer, records)
  uint32_t grid = 0;           // co-resident work-groups of moe_decode
  float *hc_n = nullptr, *hc_l = nullptr, *hc_x = nullptr;  // the hyper-connection mix's scratch (hc_lr > 0)
  uint32_t *cnt_hc = nullptr;
  float *hc_R_stage = nullptr;  // moe_forward_hc's device copy of R (max_tokens tokens)
  HcBufs hcp{};                 // the prefill mix's scratch (hc_lr > 0 and max_tokens > the decode kernel's)
  uint8_t *codebooks = nullptr;  // the caller's iq2s_grid and iq3xxs_grid (QGRID layout, up to QGRID_IQ3S)
  bool have_codebooks = false;
  const void *kernel = nullptr;  // moe_decode for the context's set of weight types
  const void *kernel_hc = nullptr;  // the same with the hyper-connection items (hc_lr > 0)
  uint32_t grid_hc = 0;
  uint32_t grid_fit = 0, grid_hc_fit = 0;  // what the device holds at once (moe_set_grid(0) returns to them)
  size_t lds_hc = 0;
  size_t lds = 0;              // its dynamic LDS
  int timing = 0;  // 0 off, 1 every kernel, 2 the decode kernel and the prefill gate/up launches
  uint64_t *trace = nullptr;   // per-item stamps of the last forward, when tracing
  uint32_t trace_cap = 0, last_T = 0, last_route = 1;
  bool last_hc = false;
  std::vector<hipEvent_t> ev;  // the event pool
  size_t ev_next = 0;          // events of the pool in use by the record
  std::vector<TimedLaunch> timed;
  std::vector<TimedSum> timed_sums;  // launches folded out of `timed`
  uint32_t ev_used = 0;        // forwards recorded since the last moe_kernel_times
  std::vector<void *> allocs;
  uint64_t dev_bytes = 0;
  std::string err;

  template <typename T>
  T *alloc(uint64_t count) {
    void *p = nullptr;
    const uint64_t bytes = std::max<uint64_t>(count * sizeof(T), 256);
    check(hipMalloc(&p, bytes), "hipMalloc");
    allocs.push_back(p);
    dev_bytes += bytes;
    return (T *)p;
  }
};

namespace {

moe_status fail(moe_ctx *c, const Error &e) {
  if (c) c->err = e.what();
  return e.st;
}

thread_local std::string g_open_error;

template <typename F>
moe_status guarded(moe_ctx *c, F f) {
  if (!c) return MOE_BAD_ARGUMENT;
  try {
    f();
    c->err.clear();
    return MOE_OK;
  } catch (const Error &e) {
    return fail(c, e);
  } catch (const std::bad_alloc &) {
    c->err = "out of host memory";
    return MOE_ERROR;
  } catch (const std::exception &e) {
    c->err = e.what();
    return MOE_ERROR;
  }
}

void validate(const moe_config &c) {
  require(c.n_embd && c.n_embd % 512 == 0 && c.n_embd / kUnit <= kMaxUnits, "n_embd must be a multiple of 512, at most 8192");
  require(c.n_ff && c.n_ff % 64 == 0 && units_of(c.n_ff) <= kMaxUnits, "n_ff must be a multiple of 64, at most 8192");
  const auto down_ok = [&](uint32_t t) { return c.n_ff % quant_block_values(t) == 0; };
  require(down_ok(c.down_type) && (!c.has_shared || down_ok(c.sh_down_type)),
          "n_ff must be a whole number of the down type's blocks (64 for Q2_0, 256 for Q4_K and IQ3_S)");
  require(c.n_ff % gate_up_rows(unit_lanes(units_of(c.n_embd))) == 0 &&
              c.n_embd % down_rows(unit_lanes(units_of(c.n_ff))) == 0,
          "n_ff and n_embd must be whole numbers of the decode kernel's row blocks");
  require(c.n_expert && c.n_expert <= kMaxExperts, "n_expert must be 1..512");
  require(c.n_used && c.n_used <= kMaxUsed && c.n_used <= c.n_expert, "n_used must be 1..min(16, n_expert)");
  const char *kTypes = "Q8_0, Q4_K, Q5_K, Q6_K, IQ3_S, IQ4_NL, IQ4_XS, Q2_0, IQ3_XXS or IQ2_S";
  require(quant_gpu_supported(c.gate_type) && quant_gpu_supported(c.down_type),
          std::string("expert types must be ") + kTypes);
  if (c.has_shared) {
    require(quant_gpu_supported(c.sh_gate_type) && quant_gpu_supported(c.sh_up_type) &&
                quant_gpu_supported(c.sh_down_type),
            std::string("shared expert types must be ") + kTypes);
    require(c.sh_up_type == c.sh_gate_type ||
                (quant_vec_dot_type(c.sh_up_type) == quant_vec_dot_type(c.sh_gate_type) &&
                 !grid_family(c.sh_gate_type) && !grid_family(c.sh_up_type)),
            "the shared expert's gate and up may differ only among types of one activation type without a codebook");
    require(c.sh_up_type == c.sh_gate_type || c.n_ff % 128 == 0,
            "a shared expert with gate and up of different types needs n_ff a multiple of 128");
  }
  require(c.max_tokens <= kMaxPrefillTokens, "max_tokens must be at most 16384");
  require(c.swiglu_limit >= 0.0f, "swiglu_limit must be >= 0");
  require(c.hc_lr <= kHcMaxLr && c.hc_lr % 8 == 0, "hc_lr must be a multiple of 8, at most 512");
}

// Types that decode through the caller's codebooks need them set first.
void need_codebooks(const moe_ctx *c, std::initializer_list<uint32_t> types) {
  for (uint32_t t : types)
    require(!quant_needs_codebook(t) || c->have_codebooks,
            "IQ3_XXS and IQ2_S weights need ggml's codebooks: call moe_set_codebooks first");
}

DecodeParams base_params(moe_ctx *c, uint32_t layer, uint32_t T) {
  const moe_config &g = c->cfg;
  need_codebooks(c, {g.gate_type, g.down_type, g.has_shared ? g.sh_gate_type : 0u, g.has_shared ? g.sh_up_type : 0u,
                     g.has_shared ? g.sh_down_type : 0u});
  const Layer &L = c->layers[layer];
  DecodeParams p{};
  p.H = g.n_embd, p.F = g.n_ff, p.E = g.n_expert, p.K = g.n_used, p.T = T;
  p.gate_type = g.gate_type, p.down_type = g.down_type;
  p.sh_gate_type = g.sh_gate_type, p.sh_down_type = g.sh_down_type, p.has_shared = g.has_shared;
  p.sh_up_type = g.sh_up_type;
  p.xact_r = quant_vec_dot_type(g.gate_type);
  p.xact_s = g.has_shared ? quant_vec_dot_type(g.sh_gate_type) : p.xact_r;
  p.swiglu_limit = g.swiglu_limit;
  p.route = 1;
  p.router = L.router, p.bias = L.has_bias ? L.bias : nullptr;
  p.experts = L.experts, p.ex_bytes = c->ex_bytes, p.ex_up_off = c->ex_up, p.ex_down_off = c->ex_down;
  p.shared = L.shared, p.sh_up_off = c->sh_up, p.sh_down_off = c->sh_down;
  p.act_r = c->act_r, p.act_s = p.xact_s == p.xact_r ? c->act_r : c->act_s;
  p.codebooks = c->codebooks;
  if (L.has_miss) {
    require(c->miss_dev != nullptr, "the layer has experts off the device: call moe_miss_buffers first");
    p.resident = L.resident;
    p.miss_jobs = c->miss_dev, p.miss_stride = (uint32_t)c->miss_stride;
    p.ans_y = (const float *)(c->miss_dev + c->miss_stride * c->tdec);
    p.ans_seq = (const uint32_t *)(c->miss_dev + c->miss_stride * c->tdec + (uint64_t)c->tdec * g.n_embd * 4);
  }
  p.logits = c->logits, p.ids = c->ids, p.w = c->w, p.gs = c->gs, p.ids_t = c->ids_t, p.w_t = c->w_t;
  p.groups = c->groups, p.ngroups = c->ngroups;
  p.h = c->h, p.y_asg = c->y_asg;
  p.flags = c->flags, p.err = c->err_flag;
  p.cnt_route = c->cnt_route, p.cnt_topk = c->cnt_topk;
  p.cnt_dyn = c->cnt_dyn;
  return p;
}

// Records an event on s for a timed launch (start or end), from the context's pool.
hipEvent_t timing_event(moe_ctx *c, hipStream_t s) {
  if (c->ev_next == c->ev.size()) {
    hipEvent_t e;
    check(hipEventCreate(&e), "hipEventCreate");
    c->ev.push_back(e);
  }
  hipEvent_t e = c->ev[c->ev_next++];
  check(hipEventRecord(e, s), "hipEventRecord");
  return e;
}
// Waits for the recorded launches and adds their durations to the per-kernel sums; the pool is then free again.
void fold_timed(moe_ctx *c) {
  if (c->timed.empty()) return;
  check(hipEventSynchronize(c->timed.back().b), "hipEventSynchronize");
  for (const TimedLaunch &t : c->timed) {
    size_t i = 0;
    while (i < c->timed_sums.size() && std::strcmp(c->timed_sums[i].name, t.name) != 0) i++;
    if (i == c->timed_sums.size()) c->timed_sums.push_back(TimedSum{t.name, 0.0, 0});
    float ms = 0.0f;
    check(hipEventElapsedTime(&ms, t.a, t.b), "hipEventElapsedTime");
    c->timed_sums[i].ms += ms, c->timed_sums[i].n++;
  }
  c->timed.clear();
  c->ev_next = 0;
}

void timing_hook(void *ctx, const char *name, int after, hipStream_t s) {
  moe_ctx *c = (moe_ctx *)ctx;
  if (c->timing == 2 && std::strcmp(name, "moe_decode") != 0 && std::strncmp(name, "pf_gate_up", 10) != 0) return;
  if (!after && c->timed.size() >= kTimedFold) fold_timed(c);
  if (!after) {
    c->timed.push_back(TimedLaunch{name, timing_event(c, s), nullptr});
  } else {
    c->timed.back().b = timing_event(c, s);
  }
}

// Zeroes the tagged-record buffers (tag 0 is never a launch's) and the list counters.
void clear_tagged(moe_ctx *c, hipStream_t s) {
  for (const auto &b : c->tagged) check(hipMemsetAsync(b.first, 0, b.second * sizeof(uint64_t), s), "hipMemsetAsync");
}

void launch(moe_ctx *c, const DecodeParams &p, hipStream_t s) {
  DecodeParams q = p;
  q.epoch = ++c->epoch;
  if ((uint32_t)q.epoch == 0) {  // the 32-bit tags wrap (every 2^32 launches): old records must not match
    clear_tagged(c, s);
    q.epoch = ++c->epoch;
  }
  q.tag = (uint32_t)q.epoch;
  c->last_step = q.tag;
  if (c->trace) q.trace = c->trace, q.trace_cap = c->trace_cap;
  c->last_T = p.T, c->last_route = p.route, c->last_hc = p.hc_R != nullptr;
  if (c->timing) timing_hook(c, "moe_decode", 0, s);
  void *args[] = {&q};
  if (q.hc_R)
    check(hipLaunchKernel(c->kernel_hc, dim3(c->grid_hc), dim3(kWG), args, c->lds_hc, s), "moe_decode launch");
  else
    check(hipLaunchKernel(c->kernel, dim3(c->grid), dim3(kWG), args, c->lds, s), "moe_decode launch");
  check(hipGetLastError(), "moe_decode launch");
  if (c->timing) timing_hook(c, "moe_decode", 1, s);
}

void forward_dev(moe_ctx *c, uint32_t layer, const float *x, uint32_t T, float *y, int32_t *ids, float *w,
                 hipStream_t s) {
  require(layer < c->cfg.n_layer, "layer out of range");
  require(T >= 1 && T <= c->tmax, "ntok must be 1..max_tokens");
  require(c->layers[layer].router != nullptr, "the layer's router is not loaded");
  const uint32_t K = c->cfg.n_used;
  need_codebooks(c, {c->cfg.gate_type, c->cfg.down_type, c->cfg.has_shared ? c->cfg.sh_gate_type : 0u,
                     c->cfg.has_shared ? c->cfg.sh_up_type : 0u, c->cfg.has_shared ? c->cfg.sh_down_type : 0u});
  if (T <= c->tdec) {
    DecodeParams p = base_params(c, layer, T);
    p.x = x, p.y = y;
    launch(c, p, s);
    c->last_ids = c->ids, c->last_w = c->w;
  } else {
    const moe_config &g = c->cfg;
    const Layer &L = c->layers[layer];
    require(!L.has_miss, "the prefill path takes only layers whose experts are all on the device (moe_set_resident)");
    PfShape S{g.n_embd, g.n_ff, g.n_expert, K, T, g.gate_type, g.down_type, g.sh_gate_type, g.sh_down_type,
              g.has_shared, g.swiglu_limit, g.sh_up_type, (g.flags & MOE_FLAG_EXACT_ROUTER) ? 1u : 0u};
    PfLayer PL{L.router, L.router_t, L.has_bias ? L.bias : nullptr, L.experts, c->ex_bytes, c->ex_up, c->ex_down, L.shared,
               c->sh_up, c->sh_down, c->codebooks, L.rlsb, L.rmax, L.bias_max};
    PfHook hook{c->timing ? timing_hook : nullptr, c};
    check(prefill_forward(S, PL, c->pf, x, y, s, hook), "prefill launch");
    c->last_ids = c->pf.ids, c->last_w = c->pf.w, c->last_pf_T = T;
  }
  if (c->timing) c->ev_used++;
  if (ids) check(hipMemcpyAsync(ids, c->last_ids, sizeof(int32_t) * T * K, hipMemcpyDeviceToDevice, s), "copy ids");
  if (w) check(hipMemcpyAsync(w, c->last_w, sizeof(float) * T * K, hipMemcpyDeviceToDevice, s), "copy w");
}

// A wait inside moe_decode gave up: its result is not to be trusted. The caller has synchronised the stream the
// forward ran on.
void check_err(moe_ctx *c) {
  uint32_t e = 0;
  check(hipMemcpy(&e, c->err_flag, 4, hipMemcpyDeviceToHost), "read error flag");
  if (e) {
    (void)hipMemset(c->err_flag, 0, 4);
    throw Error(MOE_TIMEOUT, "moe_decode: a work item waited past its limit");
  }
}

// The same for the no-alloc path's error word (in the device's scratch array).
void check_err_noalloc(moe_ctx *c) {
  uint8_t *base = g_noalloc[c->cfg.device].ptr;
  if (!base || c->noalloc_bytes > kNoAllocScratchBytes) return;
  uint32_t *err = noalloc_layout(c->cfg, base).counters + 2;
  uint32_t e = 0;
  check(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost), "read error flag");
  if (e) {
    (void)hipMemset(err, 0, 4);
    throw Error(MOE_TIMEOUT, "moe_decode (no-alloc): a work item waited past its limit");
  }
}

}  // namespace

extern "C" {

MOE_API const char *moe_last_error(const moe_ctx *ctx) { return ctx ? ctx->err.c_str() : g_open_error.c_str(); }

MOE_API uint32_t moe_h_rows(const moe_config *cfg) { return cfg && cfg->n_ff % kUnit == 0 ? kUnit : 0; }

MOE_API moe_status moe_check_config(const moe_config *cfg) {
  if (!cfg) {
    g_open_error = "null argument";
    return MOE_BAD_ARGUMENT;
  }
  try {
    moe_config g = *cfg;
    if (!g.n_layer) g.n_layer = 1;
    if (!g.max_tokens) g.max_tokens = kMaxDecodeTokens;
    if (!g.sh_up_type) g.sh_up_type = g.sh_gate_type;
    validate(g);
  } catch (const Error &e) {
    g_open_error = e.what();
    return e.st;
  }
  g_open_error.clear();
  return MOE_OK;
}

MOE_API moe_status moe_open(const moe_config *cfg, moe_ctx **out) {
  if (!cfg || !out) {
    g_open_error = "null argument";
    return MOE_BAD_ARGUMENT;
  }
  *out = nullptr;
  moe_ctx *c = nullptr;
  try {
    moe_config g = *cfg;
    if (!g.n_layer) g.n_layer = 1;
    if (!g.max_tokens) g.max_tokens = kMaxDecodeTokens;
    if (!g.sh_up_type) g.sh_up_type = g.sh_gate_type;
    validate(g);
    c = new moe_ctx();
    c->cfg = g;
    int ndev = 0;
    check(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
    require(g.device >= 0 && g.device < ndev, "no such device");
    check(hipSetDevice(g.device), "hipSetDevice");
    check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
    const uint32_t H = g.n_embd, F = g.n_ff, E = g.n_expert;
    const uint64_t gu = matrix_bytes(g.gate_type, F, H), dn = matrix_bytes(g.down_type, H, F);
    c->ex_up = gu, c->ex_down = 2 * gu, c->ex_bytes = 2 * gu + dn;
    if (g.has_shared) {
      const uint64_t sg = matrix_bytes(g.sh_gate_type, F, H), su = matrix_bytes(g.sh_up_type, F, H);
      const uint64_t sdn = matrix_bytes(g.sh_down_type, H, F);
      c->sh_up = sg, c->sh_down = sg + su, c->sh_bytes = sg + su + sdn;
    }
    c->layers.resize(g.n_layer);
    for (auto &L : c->layers) {
      L.router = c->alloc<uint16_t>((uint64_t)(E + 1) * H);
      L.bias = c->alloc<float>(E);
      L.rlsb = c->alloc<int>(E);
      L.router_t = c->alloc<uint16_t>((uint64_t)(E + 15) / 16 * 16 * H);
      L.resident = c->alloc<uint8_t>(E);
      L.experts = c->alloc<uint8_t>(c->ex_bytes * E);
      if (g.has_shared) L.shared = c->alloc<uint8_t>(c->sh_bytes);
      check(hipMemset(L.experts, 0, c->ex_bytes * E), "hipMemset");
      check(hipMemset(L.resident, 1, E), "hipMemset");
      if (L.shared) check(hipMemset(L.shared, 0, c->sh_bytes), "hipMemset");
      if (g.hc_lr) {
        L.hc_gamma = c->alloc<float>((uint64_t)kHcStreams * H);
        L.hc_down = c->alloc<uint16_t>((uint64_t)g.hc_lr * kHcStreams * H);
        L.hc_inj = c->alloc<uint16_t>((uint64_t)kHcStreams * kHcStreams * H);
        L.hc_up = c->alloc<uint16_t>((uint64_t)kHcStreams * H * g.hc_lr);
        L.hc_rn = c->alloc<double>((uint64_t)g.hc_lr + kHcStreams + (uint64_t)kHcStreams * H);
        L.hc_rlsb = c->alloc<int>((uint64_t)g.hc_lr + kHcStreams + (uint64_t)kHcStreams * H);
      }
    }
    // Scratch for max_tokens tokens of n_used + 1 assignments (the pre-routed path may give a token its shared
    // expert as a job).
    const uint32_t TM = g.max_tokens, T = std::min<uint32_t>(TM, kMaxDecodeTokens), K1 = g.n_used + 1;
    const uint32_t G = max_groups(T, K1), A = T * K1 + T;
    c->tmax = TM, c->tdec = T, c->k1 = K1, c->gmax = G;
    const uint32_t Ug = units_of(H), Ud = units_of(F);
    c->x_dev = c->alloc<float>((uint64_t)TM * H);
    c->y_dev = c->alloc<float>((uint64_t)TM * H);
    c->ids_stage = c->alloc<int32_t>((uint64_t)T * K1);
    c->w_stage = c->alloc<float>((uint64_t)T * K1);
    if (TM > T) {  // the prefill path's scratch (a pre-routed call's token may take n_used + 1 jobs)
      const uint32_t K = g.n_used + 1;
      const uint64_t A2 = (uint64_t)TM * K;
      PfBufs &b = c->pf;
      b.act_r = c->alloc<uint8_t>((uint64_t)TM * Ug * kActBytes);
      b.act_s = quant_vec_dot_type(g.sh_gate_type) != quant_vec_dot_type(g.gate_type) && g.has_shared
                    ? c->alloc<uint8_t>((uint64_t)TM * Ug * kActBytes)
                    : b.act_r;
      b.logits = c->alloc<float>((uint64_t)TM * (E + 1));
      b.xb = c->alloc<uint16_t>((uint64_t)TM * H);
      b.xt = c->alloc<uint16_t>((uint64_t)(TM + 15) / 16 * 16 * H);
      b.xn = c->alloc<float>(TM);
      b.xlsb = c->alloc<int>(TM);
      b.cnt_exact = c->alloc<uint32_t>(1);
      check(hipMemset(b.cnt_exact, 0, sizeof(uint32_t)), "hipMemset");
      b.ids = c->alloc<int32_t>(A2);
      b.w = c->alloc<float>(A2);
      b.gs = c->alloc<float>(TM);
      b.perm = c->alloc<uint32_t>(A2);
      b.inv = c->alloc<uint32_t>(A2);
      // Up to kMaxExperts experts: a layer's, or a pre-routed call's borrowed ones.
      b.tiles = c->alloc<MoeTile>(pf_max_tiles(TM, K, kMaxExperts));
      b.ntiles = c->alloc<uint32_t>(1);
      b.masks = c->alloc<unsigned long long>((uint64_t)pf_windows(TM) * kMaxExperts);
      b.h = c->alloc<float>(A2 * F);
      b.hact = c->alloc<uint8_t>(A2 * Ud * kActBytes);
      b.y_asg = c->alloc<float>(A2 * H);
      if (g.has_shared) {
        b.h_sh = c->alloc<float>((uint64_t)TM * F);
        if (g.sh_up_type != g.sh_gate_type) b.h_sh_up = c->alloc<float>((uint64_t)TM * F);
        b.hact_sh = c->alloc<uint8_t>((uint64_t)TM * Ud * kActBytes);
        b.y_sh = c->alloc<float>((uint64_t)TM * H);
        check(hipStreamCreateWithFlags(&b.side, hipStreamNonBlocking), "hipStreamCreate");
        check(hipEventCreateWithFlags(&b.fork, hipEventDisableTiming), "hipEventCreate");
        check(hipEventCreateWithFlags(&b.join, hipEventDisableTiming), "hipEventCreate");
        check(hipEventCreateWithFlags(&b.xq, hipEventDisableTiming), "hipEventCreate");
      }
    }
    c->act_r = c->alloc<uint8_t>((uint64_t)T * Ug * kActBytes);
    c->act_s = c->alloc<uint8_t>((uint64_t)T * Ug * kActBytes);
    c->logits = c->alloc<uint64_t>((uint64_t)T * (E + 1));
    c->ids = c->alloc<int32_t>((uint64_t)T * K1);
    c->w = c->alloc<float>((uint64_t)T * K1);
    c->gs = c->alloc<uint64_t>(T);
    c->ids_t = c->alloc<uint64_t>((uint64_t)T * K1);
    c->w_t = c->alloc<uint64_t>((uint64_t)T * K1);
    c->groups = c->alloc<MoeGroup>(G);
    c->ngroups = c->alloc<uint32_t>(1);
    c->tok_need = c->alloc<uint32_t>(T);
    // moe_decode reads h and the activation units at 32-bit byte offsets from their bases.
    require((uint64_t)A * F * sizeof(uint64_t) <= 0xffffffffull, "n_ff x assignments too large for the decode path");
    c->h = c->alloc<uint64_t>((uint64_t)A * F);
    c->y_asg = c->alloc<uint64_t>((uint64_t)A * H);
    const uint64_t ncnt = 3 + 2 * kDynLists * kDynStride + kDynStride;
    c->counters = c->alloc<uint32_t>(ncnt);
    check(hipMemset(c->counters, 0, ncnt * sizeof(uint32_t)), "hipMemset");
    c->cnt_route = c->counters;
    c->cnt_topk = c->cnt_route + 1;
    c->err_flag = c->cnt_topk + 1;
    c->cnt_dyn = c->err_flag + kDynStride;  // (a line of its own)
    c->flags = c->alloc<uint64_t>(kFlagCount);
    check(hipMemset(c->flags, 0, kFlagCount * sizeof(uint64_t)), "hipMemset");
    c->codebooks = c->alloc<uint8_t>(QGRID_IQ3S);
    if (g.hc_lr) {
      c->hc_n = c->alloc<float>((uint64_t)T * kHcStreams * H);
      c->hc_l = c->alloc<float>((uint64_t)T * (g.hc_lr + kHcStreams));
      c->hc_x = c->alloc<float>((uint64_t)T * H);
      c->cnt_hc = c->alloc<uint32_t>(2 * kDynStride);
      c->hc_R_stage = c->alloc<float>((uint64_t)TM * kHcStreams * H);
      if (TM > T) {
        const uint64_t Md = g.hc_lr + kHcStreams, D = (uint64_t)kHcStreams * H;
        HcBufs &b = c->hcp;
        b.sc = c->alloc<float>(TM * kHcStreams);
        b.nn = c->alloc<double>(TM);
        b.nlsb = c->alloc<int>(TM);
        b.llsb = c->alloc<int>(TM);
        b.part = c->alloc<double>(kHcDownSplit * TM * Md);
        b.raw = c->alloc<float>(TM * Md);
        b.open = c->alloc<uint32_t>(2 * TM * Md);
        b.open_up = c->alloc<uint32_t>(2 * TM * D);
        b.cnt = c->alloc<uint32_t>(2);
        b.lb = c->alloc<uint16_t>(TM * g.hc_lr);
        b.nb = c->alloc<uint16_t>(TM * D);
        b.ln = c->alloc<double>(TM);
        b.inj = c->alloc<float>(TM * kHcStreams);
        b.a = c->alloc<float>(TM * D);
        b.x = c->alloc<float>(TM * H);
      }
      check(hipMemset(c->cnt_hc, 0, 2 * kDynStride * sizeof(uint32_t)), "hipMemset");
    }
    c->tagged = {{c->logits, (uint64_t)T * (E + 1)}, {c->gs, T}, {c->ids_t, (uint64_t)T * K1}, {c->w_t, (uint64_t)T * K1},
                 {c->h, (uint64_t)A * F}, {c->y_asg, (uint64_t)A * H}, {(uint64_t *)c->cnt_dyn, kDynLists * kDynStride}};  // (and both sets of list counters)
    clear_tagged(c, nullptr);
    // The grid: every work-group the device holds at once (no more, so that all run together), LDS for the largest
    // stage.
    const size_t hc_lds = g.hc_lr ? ((size_t)T * g.hc_lr + (size_t)T * kHcStreams * kHcUpValues) * 4 : 0;
    c->lds = std::max<size_t>({(size_t)MOE_GROUP_MAX * act_tok_stride(Ug) +
                                   std::max<size_t>(Ug == 8 ? kMfmaXchBytes : 0, gate_up_xch_bytes(unit_lanes(Ug))),
                               (size_t)MOE_GROUP_MAX * act_tok_stride(Ud), kGroupingLds, kRouterLds});
    int per_cu = 0, ncu = 0;
    uint32_t types = type_bit(g.gate_type) | type_bit(g.down_type);
    if (g.has_shared) types |= type_bit(g.sh_gate_type) | type_bit(g.sh_up_type) | type_bit(g.sh_down_type);
    c->kernel = decode_kernel(types, false);
    check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, c->kernel, kWG, c->lds), "occupancy");
    check(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, g.device), "CU count");
    require(per_cu >= 1, "moe_decode does not fit a CU");
    if (const char *e = std::getenv("C0VEN_DECODE_WG_PER_CU")) per_cu = std::max(1, std::min(per_cu, std::atoi(e)));
    c->grid = c->grid_fit = (uint32_t)(per_cu * ncu);
    if (g.hc_lr) {  // the variant with the hyper-connection items: its own occupancy (every work-group resident)
      c->kernel_hc = decode_kernel(types, true);
      c->lds_hc = std::max(c->lds, hc_lds);
      int hc_per_cu = 0;
      check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&hc_per_cu, c->kernel_hc, kWG, c->lds_hc), "occupancy");
      require(hc_per_cu >= 1, "moe_decode with the hyper-connection items does not fit a CU");
      c->grid_hc = c->grid_hc_fit = (uint32_t)(std::min(hc_per_cu, per_cu) * ncu);
    }
    require(g.device < kMaxDevices, "device ordinal too large");
    noalloc_setup(g.device);
    c->noalloc_bytes = noalloc_layout(g, nullptr).bytes;
    check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    *out = c;
    return MOE_OK;
  } catch (const Error &e) {
    g_open_error = e.what();
    moe_close(c);
    return e.st;
  } catch (const std::exception &e) {
    g_open_error = e.what();
    moe_close(c);
    return MOE_ERROR;
  }
}

MOE_API void moe_close(moe_ctx *c) {
  if (!c) return;
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  if (c->pf.side) (void)hipStreamSynchronize(c->pf.side);
  for (void *p : c->allocs) (void)hipFree(p);
  for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
  if (c->pf.fork) (void)hipEventDestroy(c->pf.fork);
  if (c->pf.join) (void)hipEventDestroy(c->pf.join);
  if (c->pf.xq) (void)hipEventDestroy(c->pf.xq);
  if (c->pf.side) (void)hipStreamDestroy(c->pf.side);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  if (c->miss_host) (void)hipHostFree(c->miss_host);
  delete c;
}

MOE_API moe_status moe_load_router(moe_ctx *c, uint32_t layer, const uint16_t *router, const float *bias) {
  return guarded(c, [&] {
    require(layer < c->cfg.n_layer && router, "bad layer or null router");
    Layer &L = c->layers[layer];
    const uint64_t n = (uint64_t)(c->cfg.n_expert + 1) * c->cfg.n_embd;
    check(hipMemcpy(L.router, router, n * sizeof(uint16_t), hipMemcpyHostToDevice), "upload router");
    L.has_bias = bias != nullptr;
    if (bias) check(hipMemcpy(L.bias, bias, c->cfg.n_expert * sizeof(float), hipMemcpyHostToDevice), "upload bias");
    // The prefill router's bound: max ||W_e||_2 over the routed rows and max |bias|, rounded up.
    double r2 = 0.0;
    for (uint32_t e = 0; e < c->cfg.n_expert; e++) {
      double s2 = 0.0;
      for (uint32_t k = 0; k < c->cfg.n_embd; k++) {
        uint32_t u = (uint32_t)router[(uint64_t)e * c->cfg.n_embd + k] << 16;
        float f;
        std::memcpy(&f, &u, 4);
        s2 += (double)f * (double)f;
      }
      r2 = std::max(r2, s2);
    }
    L.rmax = (float)(std::sqrt(r2) * (1.0 + 1e-9)) * (1.0f + 0x1p-22f);
    std::vector<int> lsb(c->cfg.n_expert, 1 << 20);
    for (uint32_t e = 0; e < c->cfg.n_expert; e++)
      for (uint32_t k = 0; k < c->cfg.n_embd; k++) {
        const uint32_t b = router[(uint64_t)e * c->cfg.n_embd + k], ex = (b >> 7) & 0xffu;
        if (b & 0x7fffu) lsb[e] = std::min(lsb[e], ex == 0 ? -133 : (int)ex - 134);
      }
    check(hipMemcpy(L.rlsb, lsb.data(), lsb.size() * sizeof(int), hipMemcpyHostToDevice), "upload row lsb");
    // The routed rows in 16 x 32 tiles: tile (row / 16, k / 32) at ((row / 16) (H / 32) + k / 32) 512, a row's 32
    // values contiguous inside it.
    const uint32_t H = c->cfg.n_embd, E = c->cfg.n_expert;
    std::vector<uint16_t> tiled((uint64_t)(E + 15) / 16 * 16 * H, 0);
    for (uint32_t e = 0; e < E; e++)
      for (uint32_t k = 0; k < H; k++)
        tiled[((uint64_t)(e / 16) * (H / 32) + k / 32) * 512 + (e % 16) * 32 + k % 32] = router[(uint64_t)e * H + k];
    check(hipMemcpy(L.router_t, tiled.data(), tiled.size() * 2, hipMemcpyHostToDevice), "upload tiled router");
    L.bias_max = 0.0f;
    if (bias)
      for (uint32_t e = 0; e < c->cfg.n_expert; e++) L.bias_max = std::max(L.bias_max, std::fabs(bias[e]));
  });
}

MOE_API moe_status moe_load_expert(moe_ctx *c, uint32_t layer, uint32_t expert, const uint8_t *gate, const uint8_t *up,
                                   const uint8_t *down) {
  return guarded(c, [&] {
    const moe_config &g = c->cfg;
    require(layer < g.n_layer && gate && up && down, "bad layer or null matrix");
    const bool shared = expert == g.n_expert;
    require(expert < g.n_expert || (shared && g.has_shared), "expert out of range");
    const uint32_t gt = shared ? g.sh_gate_type : g.gate_type, ut = shared ? g.sh_up_type : g.gate_type;
    const uint32_t dt = shared ? g.sh_down_type : g.down_type;
    const uint64_t gb = matrix_bytes(gt, g.n_ff, g.n_embd), ub = matrix_bytes(ut, g.n_ff, g.n_embd);
    const uint64_t dn = matrix_bytes(dt, g.n_embd, g.n_ff);
    std::vector<uint8_t> buf(gb + ub + dn);
    repack_matrix(gt, gate, g.n_ff, g.n_embd, buf.data());
    repack_matrix(ut, up, g.n_ff, g.n_embd, buf.data() + gb);
    repack_matrix(dt, down, g.n_embd, g.n_ff, buf.data() + gb + ub);
    uint8_t *dst = shared ? c->layers[layer].shared : c->layers[layer].experts + (uint64_t)expert * c->ex_bytes;
    check(hipMemcpy(dst, buf.data(), buf.size(), hipMemcpyHostToDevice), "upload expert");
  });
}

MOE_API moe_status moe_load_layer_gguf(moe_ctx *c, uint32_t layer, const c0ven_gguf *file, uint32_t blk) {
  return guarded(c, [&] {
    const moe_config &g = c->cfg;
    require(file != nullptr && layer < g.n_layer, "null file or layer out of range");
    const uint64_t H = g.n_embd, F = g.n_ff, E = g.n_expert;
    const std::string pre = "blk." + std::to_string(blk) + ".";
    // The tensor of a name with the given type and shape (ggml order), or an error naming what differs.
    const auto tensor = [&](const std::string &name, uint32_t type, std::initializer_list<uint64_t> shape) {
      const gguf_tensor_info *tp = file->ix.tensor((pre + name).c_str());
      require(tp != nullptr, "the file has no tensor " + pre + name);
      const gguf_tensor_info &t = *tp;
      bool same = t.type == type && t.n_dims == shape.size();
      uint32_t d = 0;
      for (uint64_t v : shape) same = same && t.shape[d++] == v;
      require(same, pre + name + ": type " + std::to_string(t.type) + " or shape differs from the context's (type " +
                        std::to_string(type) + ")");
      return t.data;
    };
    // The router: n_expert rows of n_embd bf16, then the shared expert's gate row (zero without a shared expert).
    std::vector<uint16_t> router((E + 1) * H, 0);
    std::memcpy(router.data(), tensor("ffn_gate_inp.weight", QT_BF16, {H, E}), E * H * 2);
    if (g.has_shared) std::memcpy(router.data() + E * H, tensor("ffn_gate_inp_shexp.weight", QT_BF16, {H}), H * 2);
    if (moe_load_router(c, layer, router.data(), nullptr) != MOE_OK) throw Error(MOE_ERROR, c->err);
    const uint8_t *gate = tensor("ffn_gate_exps.weight", g.gate_type, {H, F, E});
    const uint8_t *up = tensor("ffn_up_exps.weight", g.gate_type, {H, F, E});
    const uint8_t *down = tensor("ffn_down_exps.weight", g.down_type, {F, H, E});
    const uint64_t gb = F * gguf_type_bytes(g.gate_type, H), db = H * gguf_type_bytes(g.down_type, F);
    for (uint32_t e = 0; e < E; e++)
      if (moe_load_expert(c, layer, e, gate + e * gb, up + e * gb, down + e * db) != MOE_OK)
        throw Error(MOE_ERROR, c->err);
    if (g.has_shared) {
      const uint8_t *sg = tensor("ffn_gate_shexp.weight", g.sh_gate_type, {H, F});
      const uint8_t *su = tensor("ffn_up_shexp.weight", g.sh_up_type, {H, F});
      const uint8_t *sd = tensor("ffn_down_shexp.weight", g.sh_down_type, {F, H});
      if (moe_load_expert(c, layer, (uint32_t)E, sg, su, sd) != MOE_OK) throw Error(MOE_ERROR, c->err);
    }
  });
}

MOE_API moe_status moe_forward(moe_ctx *c, uint32_t layer, const float *x, uint32_t ntok, uint64_t x_stride, float *y,
                               uint64_t y_stride, moe_route_out *route) {
  return guarded(c, [&] {
    require(x && y && ntok >= 1 && ntok <= c->tmax, "bad x, y or ntok");
    const uint32_t H = c->cfg.n_embd, K = c->cfg.n_used;
    require(x_stride >= H && y_stride >= H, "strides below n_embd");
    check(hipMemcpy2DAsync(c->x_dev, H * sizeof(float), x, x_stride * sizeof(float), H * sizeof(float), ntok,
                           hipMemcpyHostToDevice, c->stream),
          "upload x");
    forward_dev(c, layer, c->x_dev, ntok, c->y_dev, nullptr, nullptr, c->stream);
    check(hipMemcpy2DAsync(y, y_stride * sizeof(float), c->y_dev, H * sizeof(float), H * sizeof(float), ntok,
                           hipMemcpyDeviceToHost, c->stream),
          "download y");
    if (route && route->ids)
      check(hipMemcpyAsync(route->ids, c->last_ids, sizeof(int32_t) * ntok * K, hipMemcpyDeviceToHost, c->stream),
            "ids");
    if (route && route->w)
      check(hipMemcpyAsync(route->w, c->last_w, sizeof(float) * ntok * K, hipMemcpyDeviceToHost, c->stream), "w");
    check(hipStreamSynchronize(c->stream), "forward");
    check_err(c);
  });
}

MOE_API moe_status moe_forward_async(moe_ctx *c, uint32_t layer, const float *x_dev, uint32_t ntok, float *y_dev,
                                     int32_t *ids_dev, float *w_dev, void *stream) {
  return guarded(c, [&] {
    require(x_dev && y_dev, "null x or y");
    require((((uintptr_t)x_dev | (uintptr_t)y_dev) & 15u) == 0, "x and y must be 16-byte aligned");
    forward_dev(c, layer, x_dev, ntok, y_dev, ids_dev, w_dev, stream ? (hipStream_t)stream : c->stream);
  });
}

MOE_API moe_status moe_load_hc(moe_ctx *c, uint32_t layer, const float *gamma, const uint16_t *w_down,
                               const uint16_t *w_inject, const uint16_t *w_up) {
  return guarded(c, [&] {
    const moe_config &g = c->cfg;
    require(g.hc_lr > 0, "the context has no hyper-connection module (hc_lr = 0)");
    require(layer < g.n_layer && gamma && w_down && w_inject && w_up, "bad layer or null tensor");
    Layer &L = c->layers[layer];
    const uint64_t D = (uint64_t)kHcStreams * g.n_embd;
    check(hipMemcpy(L.hc_gamma, gamma, D * sizeof(float), hipMemcpyHostToDevice), "upload hc gamma");
    check(hipMemcpy(L.hc_down, w_down, (uint64_t)g.hc_lr * D * 2, hipMemcpyHostToDevice), "upload hc down");
    check(hipMemcpy(L.hc_inj, w_inject, (uint64_t)kHcStreams * D * 2, hipMemcpyHostToDevice), "upload hc inject");
    check(hipMemcpy(L.hc_up, w_up, D * g.hc_lr * 2, hipMemcpyHostToDevice), "upload hc up");
    // Row 2-norms (double, rounded up) for the prefill mix's bound: W_down's, W_inject's, then W_up's rows.
    std::vector<double> rn((uint64_t)g.hc_lr + kHcStreams + D);
    const auto norm = [](const uint16_t *w, uint64_t n) {
      double ss = 0.0;
      for (uint64_t i = 0; i < n; i++) {
        uint32_t b = (uint32_t)w[i] << 16;
        float f;
        std::memcpy(&f, &b, 4);
        ss += (double)f * (double)f;
      }
      return std::sqrt(ss) * (1.0 + 0x1p-30);
    };
    std::vector<int> rl(rn.size());
    const auto lsb = [](const uint16_t *w, uint64_t n) {  // 2^(e - 134) for exponent field e; zeros add no bits
      int m = 1 << 20;
      for (uint64_t i = 0; i < n; i++)
        if (w[i] & 0x7fffu) m = std::min(m, ((w[i] >> 7) & 0xffu) == 0u ? -133 : (int)((w[i] >> 7) & 0xffu) - 134);
      return m;
    };
    for (uint32_t j = 0; j < g.hc_lr; j++) rn[j] = norm(w_down + (uint64_t)j * D, D), rl[j] = lsb(w_down + (uint64_t)j * D, D);
    for (uint32_t j = 0; j < kHcStreams; j++)
      rn[g.hc_lr + j] = norm(w_inject + (uint64_t)j * D, D), rl[g.hc_lr + j] = lsb(w_inject + (uint64_t)j * D, D);
    for (uint64_t j = 0; j < D; j++)
      rn[g.hc_lr + kHcStreams + j] = norm(w_up + j * g.hc_lr, g.hc_lr), rl[g.hc_lr + kHcStreams + j] = lsb(w_up + j * g.hc_lr, g.hc_lr);
    check(hipMemcpy(L.hc_rn, rn.data(), rn.size() * sizeof(double), hipMemcpyHostToDevice), "upload hc norms");
    check(hipMemcpy(L.hc_rlsb, rl.data(), rl.size() * sizeof(int), hipMemcpyHostToDevice), "upload hc lsb");
    L.has_hc = true;
  });
}

MOE_API moe_status moe_forward_hc_async(moe_ctx *c, uint32_t layer, float *R_dev, uint32_t ntok, float *y_dev,
                                        int32_t *ids_dev, float *w_dev, void *stream) {
  return guarded(c, [&] {
    const moe_config &g = c->cfg;
    require(R_dev != nullptr, "null R");
    require((((uintptr_t)R_dev | (uintptr_t)y_dev) & 15u) == 0, "R and y must be 16-byte aligned");
    require(layer < g.n_layer && c->layers[layer].router != nullptr, "layer out of range or its router not loaded");
    require(c->layers[layer].has_hc, "the layer's hyper-connection module is not loaded (moe_load_hc)");
    require(ntok >= 1 && ntok <= c->tmax, "moe_forward_hc_async takes 1..max_tokens tokens");
    need_codebooks(c, {g.gate_type, g.down_type, g.has_shared ? g.sh_gate_type : 0u, g.has_shared ? g.sh_up_type : 0u,
                     g.has_shared ? g.sh_down_type : 0u});
    const Layer &L = c->layers[layer];
    hipStream_t s = stream ? (hipStream_t)stream : c->stream;
    if (ntok > c->tdec) {  // the prefill path: the mix's kernels, the block, the combine's kernel
      const HcShape S{g.n_embd, g.hc_lr, ntok};
      const HcLayer HL{L.hc_gamma, L.hc_down, L.hc_inj, L.hc_up, L.hc_rn, L.hc_rlsb};
      check(prefill_hc_pre(S, HL, c->hcp, R_dev, (g.flags & MOE_FLAG_HC_FIXED_ORDER) != 0, s), "prefill hc mix launch");
      float *y = y_dev ? y_dev : c->y_dev;
      forward_dev(c, layer, c->hcp.x, ntok, y, ids_dev, w_dev, s);
      check(prefill_hc_post(S, c->hcp, R_dev, y, s), "prefill hc combine launch");
      return;
    }
    DecodeParams p = base_params(c, layer, ntok);
    p.hc_R = R_dev, p.hc_gamma = L.hc_gamma, p.hc_down = L.hc_down, p.hc_inj = L.hc_inj, p.hc_up = L.hc_up;
    p.hc_lr = g.hc_lr, p.hc_n = c->hc_n, p.hc_l = c->hc_l, p.hc_x = c->hc_x, p.cnt_hc = c->cnt_hc;
    p.x = c->hc_x, p.y = y_dev;
    launch(c, p, s);
    c->last_ids = c->ids, c->last_w = c->w;
    if (c->timing) c->ev_used++;
    const uint32_t K = g.n_used;
    if (ids_dev) check(hipMemcpyAsync(ids_dev, c->ids, sizeof(int32_t) * ntok * K, hipMemcpyDeviceToDevice, s), "ids");
    if (w_dev) check(hipMemcpyAsync(w_dev, c->w, sizeof(float) * ntok * K, hipMemcpyDeviceToDevice, s), "w");
  });
}

MOE_API moe_status moe_forward_hc(moe_ctx *c, uint32_t layer, float *R, uint32_t ntok, float *y, moe_route_out *route) {
  return guarded(c, [&] {
    require(R != nullptr && c->cfg.hc_lr > 0, "null R or no hyper-connection module");
    require(ntok >= 1 && ntok <= c->tmax, "moe_forward_hc takes 1..max_tokens tokens");
    const uint64_t rb = (uint64_t)ntok * kHcStreams * c->cfg.n_embd * sizeof(float);
    const uint32_t K = c->cfg.n_used;
    check(hipMemcpyAsync(c->hc_R_stage, R, rb, hipMemcpyHostToDevice, c->stream), "upload R");
    if (moe_forward_hc_async(c, layer, c->hc_R_stage, ntok, y ? c->y_dev : nullptr, nullptr, nullptr, c->stream) !=
        MOE_OK)
      throw Error(MOE_BAD_ARGUMENT, c->err);
    check(hipMemcpyAsync(R, c->hc_R_stage, rb, hipMemcpyDeviceToHost, c->stream), "download R");
    if (y)
      check(hipMemcpyAsync(y, c->y_dev, (uint64_t)ntok * c->cfg.n_embd * sizeof(float), hipMemcpyDeviceToHost,
                           c->stream),
            "download y");
    if (route && route->ids)
      check(hipMemcpyAsync(route->ids, c->last_ids, sizeof(int32_t) * ntok * K, hipMemcpyDeviceToHost, c->stream),
            "ids");
    if (route && route->w)
      check(hipMemcpyAsync(route->w, c->last_w, sizeof(float) * ntok * K, hipMemcpyDeviceToHost, c->stream), "w");
    check(hipStreamSynchronize(c->stream), "forward_hc");
    check_err(c);
  });
}

// The jobs of a pre-routed decode launch: the expert (its index in the weights at p.experts), the token, the weight.
struct PreJob {
  uint32_t expert, tok;
  float w;
};

// A pre-routed decode launch (ntok <= tdec) of jobs on experts at base (routed types; expert E with a shared expert:
// the context's shared expert), x and y on the device.
void decode_prerouted(moe_ctx *c, uint32_t layer, const uint8_t *base, const std::vector<PreJob> &jobs, uint32_t ntok,
                      hipStream_t s) {
  const moe_config &g = c->cfg;
  const uint32_t njobs = (uint32_t)jobs.size(), H = g.n_embd;
  std::vector<uint32_t> per(ntok, 0);
  for (const PreJob &j : jobs) per[j.tok]++;
  uint32_t K = 1;
  for (uint32_t t = 0; t < ntok; t++) K = std::max(K, per[t]);
  require(K <= c->k1, "more jobs for one token than n_used + 1");
  // Ranks in the given order per token; groups of the distinct experts in order of first job, 8 a group.
  std::vector<int32_t> ids((size_t)ntok * K, -1);
  std::vector<float> w((size_t)ntok * K, 0.0f);
  std::vector<uint32_t> asg_of(njobs), fill(ntok, 0);
  uint32_t emax = 0;
  for (uint32_t j = 0; j < njobs; j++) {
    const uint32_t t = jobs[j].tok, r = fill[t]++;
    ids[(size_t)t * K + r] = (int32_t)jobs[j].expert;
    w[(size_t)t * K + r] = jobs[j].w;
    asg_of[j] = t * K + r;
    emax = std::max(emax, jobs[j].expert);
  }
  std::vector<MoeGroup> groups;
  std::vector<uint32_t> open_group(emax + 1, UINT32_MAX);
  for (uint32_t j = 0; j < njobs; j++) {
    const uint32_t e = jobs[j].expert;
    uint32_t gi = open_group[e];
    if (gi == UINT32_MAX || groups[gi].n == MOE_GROUP_MAX) {
      MoeGroup m{};
      m.slot = (int32_t)e;
      groups.push_back(m);
      gi = open_group[e] = (uint32_t)groups.size() - 1;
    }
    groups[gi].asg[groups[gi].n++] = asg_of[j];
  }
  const uint32_t ng = (uint32_t)groups.size();
  require(ng <= max_groups(ntok, K), "too many groups");
  check(hipMemsetAsync(c->y_dev, 0, sizeof(float) * ntok * H, s), "clear y");
  if (ng) check(hipMemcpyAsync(c->groups, groups.data(), sizeof(MoeGroup) * ng, hipMemcpyHostToDevice, s), "groups");
  check(hipMemcpyAsync(c->ngroups, &ng, sizeof ng, hipMemcpyHostToDevice, s), "ngroups");
  check(hipMemcpyAsync(c->ids, ids.data(), sizeof(int32_t) * ids.size(), hipMemcpyHostToDevice, s), "ids");
  check(hipMemcpyAsync(c->w, w.data(), sizeof(float) * w.size(), hipMemcpyHostToDevice, s), "w");
  check(hipMemcpyAsync(c->tok_need, per.data(), sizeof(uint32_t) * ntok, hipMemcpyHostToDevice, s), "tok_need");
  DecodeParams p = base_params(c, layer, ntok);
  p.K = K, p.route = 0, p.has_shared = 0, p.tok_need = c->tok_need;
  p.xact_s = g.has_shared ? quant_vec_dot_type(g.sh_gate_type) : p.xact_r;
  p.act_s = p.xact_s == p.xact_r ? c->act_r : c->act_s;
  if (base != c->layers[layer].experts) {  // borrowed copies: slots 0 .. 511, none of which names the shared expert
    p.experts = base;
    p.E = kMaxExperts;
  }
  p.x = c->x_dev, p.y = c->y_dev;
  if (ng) launch(c, p, s);
  if (c->timing) c->ev_used++;
  // The host's vectors must outlive the copies above.
  check(hipStreamSynchronize(s), "pre-routed launch");
}

// One borrowed expert's three matrices (file layout) repacked into the device layout at dst (ex_bytes).
void repack_borrowed(const moe_ctx *c, const moe_expert_weights &ew, std::vector<uint8_t> &buf,
                     std::vector<uint8_t> &joined) {
  const moe_config &g = c->cfg;
  const uint32_t H = g.n_embd, F = g.n_ff;
  const uint64_t gu = c->ex_up;
  buf.resize(c->ex_bytes);
  repack_matrix(g.gate_type, ew.gate, F, H, buf.data());
  repack_matrix(g.gate_type, ew.up, F, H, buf.data() + gu);
  const uint8_t *down = ew.down;
  if (ew.down_parts == 2) {
    // The two regions joined row by row into the file's rows: part 0 of every row, then part 1 of every row.
    const uint64_t bb = quant_block_bytes(g.down_type), bv = quant_block_values(g.down_type);
    const uint64_t nb = F / bv;
    const uint64_t b0 = ew.down_blocks[0] ? ew.down_blocks[0] : nb / 2, b1 = ew.down_blocks[0] ? ew.down_blocks[1] : nb - nb / 2;
    require(b0 + b1 == nb, "down_blocks do not sum to a row");
    joined.resize(nb * bb * H);
    for (uint32_t r = 0; r < H; r++) {
      std::memcpy(joined.data() + r * nb * bb, ew.down + r * b0 * bb, b0 * bb);
      std::memcpy(joined.data() + r * nb * bb + b0 * bb, ew.down + H * b0 * bb + r * b1 * bb, b1 * bb);
    }
    down = joined.data();
  }
  repack_matrix(g.down_type, down, H, F, buf.data() + 2 * gu);
}

MOE_API moe_status moe_compute_many(moe_ctx *c, const moe_cm_job *jobs, uint32_t njobs, uint32_t ntok, const float *x,
                                    uint64_t x_stride, float *y, uint64_t y_stride) {
  return guarded(c, [&] {
    const moe_config &g = c->cfg;
    const uint32_t H = g.n_embd, F = g.n_ff;
    require(x && y && ntok >= 1 && x_stride >= H && y_stride >= H, "bad x, y, ntok or strides");
    need_codebooks(c, {g.gate_type, g.down_type, g.has_shared ? g.sh_gate_type : 0u, g.has_shared ? g.sh_up_type : 0u,
                     g.has_shared ? g.sh_down_type : 0u});
    require(ntok <= c->tdec || (ntok <= c->tmax && c->tmax > c->tdec),
            "ntok must be at most 16, or at most max_tokens when that exceeds 16");
    require(njobs == 0 || jobs, "null jobs");
    // The distinct experts by gate pointer (experts.cpp:170-177), in order of first job.
    std::vector<const uint8_t *> dg;
    std::vector<uint32_t> dj(njobs);
    std::vector<uint32_t> per(ntok, 0);
    for (uint32_t j = 0; j < njobs; j++) {
      const moe_expert_weights &ew = jobs[j].expert;
      require(ew.gate && ew.up && ew.down, "null expert matrix");
      require(jobs[j].tok < ntok, "job token out of range");
      require(ew.down_parts == 1 || ew.down_parts == 2, "down_parts must be 1 or 2");
      require(ew.down_parts == 1 || ew.down_blocks[0] || F / 2 == kUnit,
              "equal down parts are supported when each is one 256-value unit (n_ff 512)");
      require(++per[jobs[j].tok] <= c->k1, "more jobs for one token than n_used + 1");
      uint32_t d = 0;
      while (d < dg.size() && dg[d] != ew.gate) d++;
      if (d == dg.size()) dg.push_back(ew.gate);
      dj[j] = d;
    }
    const uint32_t nd = (uint32_t)dg.size();
    require(nd <= kMaxExperts, "more than 512 distinct experts in one call");
    // Device copies: grow the slots to hold this call's experts (at least 64), then map each expert to a slot.
    if (nd > c->bc_slots) {
      check(hipDeviceSynchronize(), "hipDeviceSynchronize");
      if (c->bc_base) {
        c->allocs.erase(std::find(c->allocs.begin(), c->allocs.end(), (void *)c->bc_base));
        c->dev_bytes -= (uint64_t)c->bc_slots * c->ex_bytes;
        check(hipFree(c->bc_base), "hipFree");
        c->bc_base = nullptr;
      }
      c->bc_slots = std::max<uint32_t>({nd, 64u, c->bc_slots * 2});
      c->bc_slots = std::min<uint32_t>(c->bc_slots, kMaxExperts);
      c->bc_base = c->alloc<uint8_t>((uint64_t)c->bc_slots * c->ex_bytes);
      c->bc_key.assign(c->bc_slots, nullptr);
      c->bc_used.assign(c->bc_slots, 0);
    }
    const uint64_t call = ++c->bc_calls;
    std::vector<uint32_t> slot(nd, UINT32_MAX);
    if (g.borrowed_immutable)
      for (uint32_t d = 0; d < nd; d++)
        for (uint32_t sl = 0; sl < c->bc_slots; sl++)
          if (c->bc_key[sl] == dg[d]) slot[d] = sl, c->bc_used[sl] = call;
    std::vector<uint8_t> buf, joined;
    for (uint32_t d = 0; d < nd; d++) {
      if (slot[d] != UINT32_MAX) continue;
      uint32_t best = 0;  // the least recently used slot this call has not taken
      for (uint32_t sl = 1; sl < c->bc_slots; sl++)
        if (c->bc_used[sl] < c->bc_used[best]) best = sl;
      require(c->bc_used[best] != call, "expert copies exhausted");
      slot[d] = best, c->bc_used[best] = call, c->bc_key[best] = dg[d];
      uint32_t j0 = 0;
      while (dj[j0] != d) j0++;
      repack_borrowed(c, jobs[j0].expert, buf, joined);
      check(hipMemcpy(c->bc_base + (uint64_t)best * c->ex_bytes, buf.data(), buf.size(), hipMemcpyHostToDevice),
            "upload expert");
    }
    hipStream_t s = c->stream;
    check(hipMemcpy2DAsync(c->x_dev, H * sizeof(float), x, x_stride * sizeof(float), H * sizeof(float), ntok,
                           hipMemcpyHostToDevice, s),
          "upload x");
    std::vector<PreJob> pj(njobs);
    for (uint32_t j = 0; j < njobs; j++) pj[j] = PreJob{slot[dj[j]], jobs[j].tok, jobs[j].w};
    if (njobs == 0) {
      check(hipMemsetAsync(c->y_dev, 0, sizeof(float) * ntok * H, s), "clear y");
    } else if (ntok <= c->tdec) {
      decode_prerouted(c, 0, c->bc_base, pj, ntok, s);
    } else {
      uint32_t K = 1;
      for (uint32_t t = 0; t < ntok; t++) K = std::max(K, per[t]);
      std::vector<int32_t> ids((size_t)ntok * K, -1);
      std::vector<float> w((size_t)ntok * K, 0.0f);
      std::vector<uint32_t> fill(ntok, 0);
      for (const PreJob &q : pj) {
        const uint32_t r = fill[q.tok]++;
        ids[(size_t)q.tok * K + r] = (int32_t)q.expert, w[(size_t)q.tok * K + r] = q.w;
      }
      check(hipMemcpyAsync(c->pf.ids, ids.data(), sizeof(int32_t) * ids.size(), hipMemcpyHostToDevice, s), "ids");
      check(hipMemcpyAsync(c->pf.w, w.data(), sizeof(float) * w.size(), hipMemcpyHostToDevice, s), "w");
      PfShape S{H, F, c->bc_slots, K, ntok, g.gate_type, g.down_type, g.sh_gate_type, g.sh_down_type, 0, g.swiglu_limit,
                g.sh_up_type};
      PfLayer PL{nullptr, nullptr, nullptr, c->bc_base, c->ex_bytes, c->ex_up, c->ex_down, nullptr, 0, 0, c->codebooks, nullptr, 0.0f, 0.0f};
      PfHook hook{c->timing ? timing_hook : nullptr, c};
      check(prefill_jobs(S, PL, c->pf, c->x_dev, c->y_dev, s, hook), "prefill launch");
      c->last_ids = c->pf.ids, c->last_w = c->pf.w, c->last_pf_T = ntok;
      check(hipStreamSynchronize(s), "pre-routed prefill");  // the host's ids and w must outlive the copies
    }
    check(hipMemcpy2DAsync(y, y_stride * sizeof(float), c->y_dev, H * sizeof(float), H * sizeof(float), ntok,
                           hipMemcpyDeviceToHost, s),
          "download y");
    check(hipStreamSynchronize(s), "compute_many");
    check_err(c);
  });
}

MOE_API moe_status moe_forward_experts(moe_ctx *c, const moe_job *jobs, uint32_t njobs, uint32_t ntok, const float *x,
                                       uint64_t x_stride, float *y, uint64_t y_stride) {
  return guarded(c, [&] {
    const moe_config &g = c->cfg;
    const uint32_t H = g.n_embd;
    require(x && y && ntok >= 1 && ntok <= c->tdec && x_stride >= H && y_stride >= H, "bad x, y, ntok or strides");
    require(njobs == 0 || jobs, "null jobs");
    const uint32_t layer = njobs ? jobs[0].layer : 0;
    std::vector<uint32_t> per(ntok, 0);
    for (uint32_t j = 0; j < njobs; j++) {
      require(jobs[j].layer == layer, "the jobs of one call must share a layer");
      require(jobs[j].tok < ntok, "job token out of range");
      require(jobs[j].expert < g.n_expert || (jobs[j].expert == g.n_expert && g.has_shared), "job expert out of range");
      per[jobs[j].tok]++;
    }
    require(layer < g.n_layer, "layer out of range");
    uint32_t K = 1;
    for (uint32_t t = 0; t < ntok; t++) K = std::max(K, per[t]);
    require(K <= c->k1, "more jobs for one token than n_used + 1");
    // Ranks in the given order per token; groups of the distinct experts in order of first job, 8 a group.
    std::vector<int32_t> ids((size_t)ntok * K, -1);
    std::vector<float> w((size_t)ntok * K, 0.0f);
    std::vector<uint32_t> asg_of(njobs), fill(ntok, 0);
    for (uint32_t j = 0; j < njobs; j++) {
      const uint32_t t = jobs[j].tok, r = fill[t]++;
      ids[(size_t)t * K + r] = (int32_t)jobs[j].expert;
      w[(size_t)t * K + r] = jobs[j].w;
      asg_of[j] = t * K + r;
    }
    std::vector<MoeGroup> groups;
    std::vector<uint32_t> open_group(g.n_expert + 1, UINT32_MAX);
    for (uint32_t j = 0; j < njobs; j++) {
      const uint32_t e = jobs[j].expert;
      uint32_t gi = open_group[e];
      if (gi == UINT32_MAX || groups[gi].n == MOE_GROUP_MAX) {
        MoeGroup m{};
        m.slot = (int32_t)e;
        groups.push_back(m);
        gi = open_group[e] = (uint32_t)groups.size() - 1;
      }
      groups[gi].asg[groups[gi].n++] = asg_of[j];
    }
    const uint32_t ng = (uint32_t)groups.size();
    require(ng <= max_groups(ntok, K), "too many groups");
    hipStream_t s = c->stream;
    check(hipMemcpy2DAsync(c->x_dev, H * sizeof(float), x, x_stride * sizeof(float), H * sizeof(float), ntok,
                           hipMemcpyHostToDevice, s),
          "upload x");
    check(hipMemsetAsync(c->y_dev, 0, sizeof(float) * ntok * H, s), "clear y");
    if (ng) check(hipMemcpyAsync(c->groups, groups.data(), sizeof(MoeGroup) * ng, hipMemcpyHostToDevice, s), "groups");
    check(hipMemcpyAsync(c->ngroups, &ng, sizeof ng, hipMemcpyHostToDevice, s), "ngroups");
    check(hipMemcpyAsync(c->ids, ids.data(), sizeof(int32_t) * ids.size(), hipMemcpyHostToDevice, s), "ids");
    check(hipMemcpyAsync(c->w, w.data(), sizeof(float) * w.size(), hipMemcpyHostToDevice, s), "w");
    check(hipMemcpyAsync(c->tok_need, per.data(), sizeof(uint32_t) * ntok, hipMemcpyHostToDevice, s), "tok_need");
    DecodeParams p = base_params(c, layer, ntok);
    p.K = K, p.route = 0, p.has_shared = 0, p.tok_need = c->tok_need;
    p.xact_s = g.has_shared ? quant_vec_dot_type(g.sh_gate_type) : p.xact_r;
    p.act_s = p.xact_s == p.xact_r ? c->act_r : c->act_s;
    p.x = c->x_dev, p.y = c->y_dev;
    if (ng) launch(c, p, s);
    if (c->timing) c->ev_used++;
    check(hipMemcpy2DAsync(y, y_stride * sizeof(float), c->y_dev, H * sizeof(float), H * sizeof(float), ntok,
                           hipMemcpyDeviceToHost, s),
          "download y");
    check(hipStreamSynchronize(s), "forward_experts");
    check_err(c);
  });
}

MOE_API moe_status moe_sync(moe_ctx *c) {
  return guarded(c, [&] {
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    check_err(c);
  });
}

MOE_API moe_status moe_check(moe_ctx *c, void *stream) {
  return guarded(c, [&] {
    check(hipStreamSynchronize(stream ? (hipStream_t)stream : c->stream), "hipStreamSynchronize");
    if (c->pf.side) check(hipStreamSynchronize(c->pf.side), "hipStreamSynchronize");
    check_err(c);
    check_err_noalloc(c);
  });
}

MOE_API moe_status moe_forward_async_noalloc(moe_ctx *c, uint32_t layer, const float *x_dev, uint32_t ntok,
                                             float *y_dev, int32_t *ids_dev, float *w_dev, void *stream) {
  return guarded(c, [&] {
    require(x_dev && y_dev, "null x or y");
    require((((uintptr_t)x_dev | (uintptr_t)y_dev) & 15u) == 0, "x and y must be 16-byte aligned");
    require(layer < c->cfg.n_layer, "layer out of range");
    require(ntok >= 1 && ntok <= c->tdec, "moe_forward_async_noalloc takes 1..min(max_tokens, 16) tokens (the decode kernel)");
    require(c->layers[layer].router != nullptr, "the layer's router is not loaded");
    require(c->noalloc_bytes <= kNoAllocScratchBytes,
            "the context's decode scratch (" + std::to_string(c->noalloc_bytes) + " B) exceeds the no-alloc array (" +
                std::to_string(kNoAllocScratchBytes) + " B)");
    NoAllocScratch &d = g_noalloc[c->cfg.device];
    require(d.ptr != nullptr, "no-alloc scratch not set up on this device");
    hipStream_t s = stream ? (hipStream_t)stream : c->stream;
    const NoAllocLayout L = noalloc_layout(c->cfg, d.ptr);
    DecodeParams p = base_params(c, layer, ntok);
    p.act_r = L.act_r, p.act_s = p.xact_s == p.xact_r ? L.act_r : L.act_s;
    p.logits = L.logits, p.ids = L.ids, p.w = L.w, p.gs = L.gs, p.ids_t = L.ids_t, p.w_t = L.w_t;
    p.groups = L.groups, p.ngroups = L.ngroups, p.h = L.h, p.y_asg = L.y_asg, p.flags = L.flags;
    p.cnt_route = L.counters, p.cnt_topk = L.counters + 1, p.err = L.counters + 2, p.cnt_dyn = L.counters + 2 + kDynStride;
    p.x = x_dev, p.y = y_dev;
    p.epoch = ++d.epoch;
    if ((uint32_t)p.epoch == 0) {  // the 32-bit tags wrap: clear the records (a fill kernel), then take the next tag
      zero_words(d.ptr, L.tagged_bytes, s);
      p.epoch = ++d.epoch;
    }
    p.tag = (uint32_t)p.epoch;
    c->last_step = p.tag;
    void *args[] = {&p};
    check(hipLaunchKernel(c->kernel, dim3(c->grid), dim3(kWG), args, c->lds, s), "moe_decode launch");
    check(hipGetLastError(), "moe_decode launch");
    const uint32_t K = c->cfg.n_used;
    if (ids_dev) check(hipMemcpyAsync(ids_dev, L.ids, sizeof(int32_t) * ntok * K, hipMemcpyDeviceToDevice, s), "copy ids");
    if (w_dev) check(hipMemcpyAsync(w_dev, L.w, sizeof(float) * ntok * K, hipMemcpyDeviceToDevice, s), "copy w");
  });
}

MOE_API void *moe_stream(moe_ctx *c) { return c ? (void *)c->stream : nullptr; }

MOE_API moe_status moe_set_timing(moe_ctx *c, int on) {
  return guarded(c, [&] {
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    require(on >= 0 && on <= 2, "timing must be 0, 1 or 2");
    c->timing = on;
    c->ev_used = 0, c->ev_next = 0;
    c->timed.clear();
    c->timed_sums.clear();
  });
}

MOE_API moe_status moe_kernel_times(moe_ctx *c, const char **names, float *avg_ms, uint32_t cap, uint32_t *n,
                                    uint32_t *forwards) {
  return guarded(c, [&] {
    require(n != nullptr, "null n");
    *n = 0;
    if (forwards) *forwards = c->ev_used;
    // Kernels in order of first launch; the average over their launches.
    fold_timed(c);
    for (size_t i = 0; i < c->timed_sums.size() && i < cap; i++) {
      if (names) names[i] = c->timed_sums[i].name;
      if (avg_ms) avg_ms[i] = (float)(c->timed_sums[i].ms / c->timed_sums[i].n);
      *n = (uint32_t)i + 1;
    }
    c->ev_used = 0, c->ev_next = 0;
    c->timed.clear();
    c->timed_sums.clear();
  });
}

MOE_API uint32_t moe_grid(const moe_ctx *c) { return c ? c->grid : 0; }

MOE_API moe_status moe_set_grid(moe_ctx *c, uint32_t grid) {
  return guarded(c, [&] {
    require(grid % 8 == 0 && grid <= (1u << 20), "the grid must be a multiple of 8 (the routed items' lists)");
    c->grid = grid ? grid : c->grid_fit;
    if (c->cfg.hc_lr) c->grid_hc = grid ? grid : c->grid_hc_fit;
  });
}

MOE_API moe_status moe_set_trace(moe_ctx *c, int on) {
  return guarded(c, [&] {
    if (on && !c->trace) {
      c->trace_cap = 1u << 16;
      c->trace = c->alloc<uint64_t>((uint64_t)4 * c->trace_cap);
    } else if (!on && c->trace) {
      check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
      c->trace = nullptr;  // the buffer stays with the context's allocations
    }
  });
}

MOE_API moe_status moe_trace(moe_ctx *c, uint64_t *stamps, uint32_t cap, uint32_t *n, uint32_t *bounds) {
  return guarded(c, [&] {
    require(n != nullptr, "null n");
    require(c->trace != nullptr, "tracing is off");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    uint32_t ng = 0;
    check(hipMemcpy(&ng, c->ngroups, 4, hipMemcpyDeviceToHost), "read ngroups");
    const moe_config &g = c->cfg;
    const uint32_t T = c->last_T, Ug = unit_lanes(units_of(g.n_embd)), Ud = unit_lanes(units_of(g.n_ff));
    const uint32_t nL = lead_items(T, g.n_expert, c->last_route), ns = shared_chunks(T, c->last_route, g.has_shared);
    const uint32_t nGU = g.n_ff / gate_up_rows(Ug), nD = g.n_embd / down_rows(Ud);
    const uint32_t nH = c->last_hc ? hc_items(T, g.n_embd, g.hc_lr) : 0;  // the hyper-connection items come first
    const uint32_t b1 = nH + nL + (c->last_route ? T : 0), b2 = b1 + ns * nGU, b3 = b2 + ns * nD, b4 = b3 + ng * nGU;
    const uint32_t b5 = b4 + ng * nD, end = b5 + T * nD;
    const uint32_t bb[8] = {nH, nH + nL, b1, b2, b3, b4, b5, end};
    if (bounds) std::memcpy(bounds, bb, sizeof bb);
    *n = std::min(end, c->trace_cap);
    if (stamps)
      check(hipMemcpy(stamps, c->trace, sizeof(uint64_t) * 4 * std::min(cap, c->trace_cap), hipMemcpyDeviceToHost),
            "download trace");
  });
}

MOE_API moe_status moe_copy_experts(moe_ctx *c, uint32_t src_layer, uint32_t dst_layer) {
  return guarded(c, [&] {
    require(src_layer < c->cfg.n_layer && dst_layer < c->cfg.n_layer, "layer out of range");
    if (src_layer == dst_layer) return;
    const Layer &a = c->layers[src_layer], &b = c->layers[dst_layer];
    check(hipMemcpy(b.experts, a.experts, c->ex_bytes * c->cfg.n_expert, hipMemcpyDeviceToDevice), "copy experts");
    if (a.shared) check(hipMemcpy(b.shared, a.shared, c->sh_bytes, hipMemcpyDeviceToDevice), "copy shared");
  });
}

MOE_API moe_status moe_expert_bytes(const moe_ctx *c, uint32_t which, uint64_t *bytes) {
  if (!c || !bytes) return MOE_BAD_ARGUMENT;
  const moe_config &g = c->cfg;
  switch (which) {
    case 0: *bytes = matrix_bytes(g.gate_type, g.n_ff, g.n_embd); break;
    case 1: *bytes = matrix_bytes(g.down_type, g.n_embd, g.n_ff); break;
    case 2: *bytes = g.has_shared ? matrix_bytes(g.sh_gate_type, g.n_ff, g.n_embd) : 0; break;
    case 3: *bytes = g.has_shared ? matrix_bytes(g.sh_down_type, g.n_embd, g.n_ff) : 0; break;
    case 4: *bytes = g.has_shared ? matrix_bytes(g.sh_up_type, g.n_ff, g.n_embd) : 0; break;
    default: return MOE_BAD_ARGUMENT;
  }
  return MOE_OK;
}

MOE_API uint64_t moe_device_bytes(const moe_ctx *c) { return c ? c->dev_bytes : 0; }

MOE_API moe_status moe_dequantize(moe_ctx *c, uint32_t type, const uint8_t *blocks, uint32_t rows, uint32_t cols,
                                  float *out) {
  return guarded(c, [&] {
    require(quant_gpu_supported(type) && blocks && out && rows && cols && cols % quant_block_values(type) == 0,
            "bad dequantize arguments");
    need_codebooks(c, {type});
    const uint64_t mb = matrix_bytes(type, rows, cols);
    std::vector<uint8_t> buf(mb);
    repack_matrix(type, blocks, rows, cols, buf.data());
    const uint32_t nrt = (rows + kTileRows - 1) / kTileRows;
    DevBuf dm, dout;
    check(hipMalloc(&dm.p, mb), "hipMalloc");
    check(hipMalloc(&dout.p, (uint64_t)nrt * kTileRows * cols * sizeof(float)), "hipMalloc");
    check(hipMemcpy(dm.p, buf.data(), mb, hipMemcpyHostToDevice), "upload");
    hipLaunchKernelGGL(moe_dequant, dim3(nrt), dim3(64), 0, c->stream, (const uint8_t *)dm.p, type, rows, cols,
                       (const uint8_t *)c->codebooks, (float *)dout.p);
    check(hipGetLastError(), "moe_dequant");
    check(hipStreamSynchronize(c->stream), "moe_dequant");
    check(hipMemcpy(out, dout.p, (uint64_t)rows * cols * sizeof(float), hipMemcpyDeviceToHost), "download");
  });
}

MOE_API moe_status moe_set_codebooks(moe_ctx *c, const uint8_t *qgrid, uint64_t bytes) {
  return guarded(c, [&] {
    require(qgrid != nullptr && bytes >= QGRID_KVALUES, "the codebook buffer must hold QGRID_IQ2S .. QGRID_KVALUES");
    // The IQ3_S region must be ggml's iq3s_grid (which this build carries): a check that the buffer has the layout.
    require(std::memcmp(qgrid + QGRID_IQ3S, kIq3sGridHost, sizeof kIq3sGridHost) == 0,
            "the buffer's IQ3_S region is not ggml's iq3s_grid: not a QGRID-layout codebook buffer");
    check(hipMemcpy(c->codebooks, qgrid, QGRID_IQ3S, hipMemcpyHostToDevice), "upload codebooks");
    c->have_codebooks = true;
  });
}

#define ROW(s, f) {#s "." #f, (uint32_t)offsetof(s, f), (uint32_t)sizeof(((s *)0)->f)}
#define STRUCT(s) {#s, 0u, (uint32_t)sizeof(s)}

MOE_API moe_status moe_prefill_dispatch(moe_ctx *c, MoeTile *tiles, uint32_t cap, uint32_t *ntiles, uint32_t *perm) {
  return guarded(c, [&] {
    require(ntiles != nullptr, "null ntiles");
    require(c->last_pf_T > 0, "no prefill forward has run");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    check(hipMemcpy(ntiles, c->pf.ntiles, 4, hipMemcpyDeviceToHost), "read ntiles");
    if (tiles && cap)
      check(hipMemcpy(tiles, c->pf.tiles, sizeof(MoeTile) * std::min(cap, *ntiles), hipMemcpyDeviceToHost), "tiles");
    if (perm)
      check(hipMemcpy(perm, c->pf.perm, sizeof(uint32_t) * c->last_pf_T * c->cfg.n_used, hipMemcpyDeviceToHost),
            "perm");
  });
}

MOE_API moe_status moe_set_resident(moe_ctx *c, uint32_t layer, const uint8_t *resident) {
  return guarded(c, [&] {
    require(layer < c->cfg.n_layer, "layer out of range");
    Layer &L = c->layers[layer];
    std::vector<uint8_t> r(c->cfg.n_expert, 1);
    if (resident)
      for (uint32_t e = 0; e < c->cfg.n_expert; e++) r[e] = resident[e] ? 1 : 0;
    check(hipMemcpy(L.resident, r.data(), r.size(), hipMemcpyHostToDevice), "upload resident flags");
    L.has_miss = std::find(r.begin(), r.end(), 0) != r.end();
  });
}

MOE_API moe_status moe_miss_buffers(moe_ctx *c, void **jobs, uint64_t *job_stride, float **ans_y, uint32_t **ans_seq) {
  return guarded(c, [&] {
    if (!c->miss_host) {
      const uint64_t stride = (sizeof(moe_miss_job) + 4ull * c->cfg.n_embd + 255) / 256 * 256;
      const uint64_t bytes = stride * c->tdec + 4ull * c->tdec * c->cfg.n_embd + 256;
      void *h = nullptr, *d = nullptr;
      check(hipHostMalloc(&h, bytes, hipHostMallocCoherent | hipHostMallocMapped), "hipHostMalloc");
      std::memset(h, 0, bytes);
      check(hipHostGetDevicePointer(&d, h, 0), "hipHostGetDevicePointer");
      c->miss_host = (uint8_t *)h, c->miss_dev = (uint8_t *)d, c->miss_stride = stride;
    }
    const uint64_t ans = c->miss_stride * c->tdec;
    if (jobs) *jobs = c->miss_host;
    if (job_stride) *job_stride = c->miss_stride;
    if (ans_y) *ans_y = (float *)(c->miss_host + ans);
    if (ans_seq) *ans_seq = (uint32_t *)(c->miss_host + ans + 4ull * c->tdec * c->cfg.n_embd);
  });
}

MOE_API uint32_t moe_last_step(const moe_ctx *c) { return c ? c->last_step : 0; }

MOE_API moe_status moe_prefill_exact_tokens(moe_ctx *c, uint32_t *n) {
  return guarded(c, [&] {
    require(n != nullptr, "null n");
    *n = 0;
    if (!c->pf.cnt_exact) return;
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    check(hipMemcpy(n, c->pf.cnt_exact, 4, hipMemcpyDeviceToHost), "read count");
    check(hipMemset(c->pf.cnt_exact, 0, 4), "clear count");
  });
}

MOE_API uint32_t moe_abi_layout(moe_abi_row *table, uint32_t cap) {
  static const moe_abi_row rows[] = {
      ROW(moe_config, n_embd),       ROW(moe_config, n_ff),         ROW(moe_config, n_expert),
      ROW(moe_config, n_used),       ROW(moe_config, n_layer),      ROW(moe_config, gate_type),
      ROW(moe_config, down_type),    ROW(moe_config, has_shared),   ROW(moe_config, sh_gate_type),
      ROW(moe_config, sh_down_type), ROW(moe_config, max_tokens),   ROW(moe_config, swiglu_limit),
      ROW(moe_config, device),       ROW(moe_config, borrowed_immutable), ROW(moe_config, hc_lr),
      ROW(moe_config, sh_up_type),   ROW(moe_config, flags),
      ROW(moe_miss_job, seq),        ROW(moe_miss_job, nmiss),      ROW(moe_miss_job, ids),
      ROW(moe_miss_job, w),          ROW(moe_miss_job, all),        STRUCT(moe_miss_job),
      STRUCT(moe_config),            ROW(moe_expert_weights, gate), ROW(moe_expert_weights, up),
      ROW(moe_expert_weights, down), ROW(moe_expert_weights, down_parts), ROW(moe_expert_weights, down_blocks),
      STRUCT(moe_expert_weights),    ROW(moe_cm_job, expert),       ROW(moe_cm_job, tok),
      ROW(moe_cm_job, w),            STRUCT(moe_cm_job),
      ROW(gguf_tensor_info, name),   ROW(gguf_tensor_info, type),   ROW(gguf_tensor_info, n_dims),
      ROW(gguf_tensor_info, shape),  ROW(gguf_tensor_info, shard),  ROW(gguf_tensor_info, offset),
      ROW(gguf_tensor_info, bytes),  ROW(gguf_tensor_info, data),   STRUCT(gguf_tensor_info),
      ROW(moe_route_out, ids),       ROW(moe_route_out, w),         STRUCT(moe_route_out),
      ROW(moe_job, layer),           ROW(moe_job, expert),          ROW(moe_job, tok),
      ROW(moe_job, w),               STRUCT(moe_job),               ROW(MoeTile, expert),
      ROW(MoeTile, slot),            ROW(MoeTile, start),           ROW(MoeTile, count),
      STRUCT(MoeTile),               ROW(MoeGroup, slot),           ROW(MoeGroup, n),
      ROW(MoeGroup, asg),            STRUCT(MoeGroup),              ROW(moe_abi_row, name),
      ROW(moe_abi_row, offset),      ROW(moe_abi_row, size),        STRUCT(moe_abi_row),
  };
  const uint32_t n = sizeof rows / sizeof rows[0];
  if (table)
    for (uint32_t i = 0; i < n && i < cap; i++) table[i] = rows[i];
  return n;
}

}  // extern "C"
