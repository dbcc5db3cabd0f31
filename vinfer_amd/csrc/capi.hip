// C ABI of the sampler library (declared in include/vsampler.h).
#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/vsampler.h"
#include "common.cuh"
#include "penalty.cuh"
#include "sample.cuh"
#include "split.cuh"
#include "uniform.h"
#include "verify.cuh"
#include "logprobs.cuh"
#include "lmhead.cuh"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(VSAMP_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_dev_ok[kMaxDevices];  // 0 unknown, 1 gfx950, 2 not
std::atomic<int> g_dev_cus[kMaxDevices];  // compute units of a checked device
// Workgroups per rejected row of a verify call, at most (the launch takes the largest power of two
// that gives every (row, slice) item a workgroup of its own: 4 for ~50 rejected rows on 256 CUs).
// Measured with the slices' fence-free hand-off (B = 192, K = 1, V = 262144): 2 slices 155.3 us
// per call, 4, 8 or 16 136.0-136.4.
constexpr int kMaxResidualSlices = 8;

int check_device(int dev, char* why, size_t n) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    if (why && n) snprintf(why, n, "no HIP device available");
    return VSAMP_E_DEVICE;
  }
  if (dev < 0 || dev >= count) {
    if (why && n) snprintf(why, n, "device %d out of range (%d devices)", dev, count);
    return VSAMP_E_DEVICE;
  }
  if (dev < kMaxDevices && g_dev_ok[dev].load() == 1) return VSAMP_OK;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) {
    if (why && n) snprintf(why, n, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    return VSAMP_E_HIP;
  }
  const bool ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  if (dev < kMaxDevices) {
    g_dev_cus[dev].store(prop.multiProcessorCount);
    g_dev_ok[dev].store(ok ? 1 : 2);
  }
  if (!ok) {
    if (why && n) snprintf(why, n, "needs a gfx950 (MI355X) GPU, device %d is %s", dev, prop.gcnArchName);
    return VSAMP_E_DEVICE;
  }
  return VSAMP_OK;
}

int check_current_device() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  char why[256];
  int rc = check_device(dev, why, sizeof why);
  if (rc) return fail(rc, "%s", why);
  return VSAMP_OK;
}

// Compute units of the current device (checked by check_current_device first).
int current_cus() {
  int dev = 0;
  const int n = hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices ? g_dev_cus[dev].load() : 0;
  return n > 0 ? n : 256;
}

size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct Layout {
  size_t n_exc, exc_id, exc_val, exc_cnt, total;
};

Layout layout(int64_t B, int64_t V, int64_t H) {
  Layout L;
  (void)V;
  size_t o = 0;
  L.n_exc = o;
  o = align_up(o + 4 * static_cast<size_t>(B));
  L.exc_id = o;
  o = align_up(o + 4 * static_cast<size_t>(H));
  L.exc_val = o;
  o = align_up(o + 4 * static_cast<size_t>(H));
  L.exc_cnt = o;
  o = align_up(o + 4 * static_cast<size_t>(H));
  L.total = o;
  return L;
}

constexpr int64_t kMaxVocab = static_cast<int64_t>(vs::kMaxStripes) * vs::kThreads * vs::kBlk;

// ---- split rows -------------------------------------------------------------------------------
// A batch of at most kSplitMaxBatch bf16 rows of at least kSplitMinVocab spreads each row over G
// workgroups of the one launch (k_sample in split mode): G = 256 / B clamped to [2, 16], so the
// launch has about 256 workgroups (one per CU) while a row's last slice merges at most 15 other
// slice records. The records, then one arrival word per row, follow the penalty part of the
// workspace.
constexpr int kSplitMaxBatch = 128;
constexpr int kSplitMinVocab = 32768;
constexpr int kSplitTarget = 256;
constexpr int kSplitMaxSlices = 16;
static_assert(kSplitMaxSlices <= vs::kMaxSlices, "slices per row");

int split_slices(int64_t B, int64_t V) {
  if (B < 1 || B > kSplitMaxBatch || V < kSplitMinVocab) return 1;
  const int64_t g = kSplitTarget / B;
  return static_cast<int>(g < 2 ? 2 : (g > kSplitMaxSlices ? kSplitMaxSlices : g));
}

// Byte offset of the slice records in the workspace (after the penalty part), and the workspace's
// size with the records and arrival words.
size_t split_records(int64_t B, int64_t V, int64_t H) { return align_up(layout(B, V, H).total); }
size_t split_total(int64_t B, int64_t V, int64_t H) {
  const int G = split_slices(B, V);
  if (G < 2) return layout(B, V, H).total;
  return split_records(B, V, H) + static_cast<size_t>(B) * G * vs::kSliceRecord + 8 * static_cast<size_t>(B);
}

// Every launch's tag for the arrival words: distinct across the launches of this process, and
// starting from a value a workspace's earlier contents are unlikely to hold.
std::atomic<uint64_t> g_epoch{(static_cast<uint64_t>(std::chrono::steady_clock::now().time_since_epoch().count()) *
                               0x9E3779B97F4A7C15ull) >> 16};
uint64_t next_epoch() { return g_epoch.fetch_add(1, std::memory_order_relaxed) & 0xFFFFFFFFFFFFull; }

// ---- the library's own workspace, for callers that cannot allocate (vsamp_sample_noalloc) ----
// 16 MiB per GPU, held from the library's first use on that GPU until the process ends: the
// workspace of histories up to ~1.39 M ids in all (4 B per row + 12 B per history id). Every
// call on one GPU shares it, so calls that overlap on one GPU (different streams, or threads)
// race. The kernels write every word of it they read within the launch (the split rows' arrival
// words are tagged with the launch), so nothing has to be cleared between calls.
constexpr size_t kScratchBytes = size_t(16) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::atomic<void*> g_scratch[kMaxDevices];  // the array's address on each device

// `scratch`'s device address on the current device (the name itself is a host-side stand-in:
// never passed to a kernel), looked up once per device.
int scratch_of_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(VSAMP_E_DEVICE, "device %d out of range", dev);
  void* p = g_scratch[dev].load();
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch[dev].store(p);
  }
  *out = p;
  return VSAMP_OK;
}

bool wants_penalties(const vsamp_args* a);

int validate(const vsamp_args* a, bool need_draw) {
  if (!a) return fail(VSAMP_E_ARG, "args is NULL");
  if (a->flags & ~(VSAMP_HIST_RANGES | VSAMP_SPLIT_ROWS | VSAMP_HIST_APPEND))
    return fail(VSAMP_E_ARG,
                "flags must be a combination of VSAMP_HIST_RANGES, VSAMP_SPLIT_ROWS and VSAMP_HIST_APPEND, got %u",
                a->flags);
  if ((a->flags & VSAMP_HIST_APPEND) && (!need_draw || !(a->flags & VSAMP_HIST_RANGES)))
    return fail(VSAMP_E_ARG, "VSAMP_HIST_APPEND goes with VSAMP_HIST_RANGES, in a call that draws");
  if ((a->flags & VSAMP_HIST_APPEND) && !wants_penalties(a))
    return fail(VSAMP_E_ARG, "VSAMP_HIST_APPEND needs penalties on (a history and a penalty column)");
  if (a->dtype != VSAMP_BF16 && a->dtype != VSAMP_F32)
    return fail(VSAMP_E_DTYPE, "unsupported logits dtype %d (VSAMP_BF16=0, VSAMP_F32=1)", a->dtype);
  if (a->batch < 0) return fail(VSAMP_E_ARG, "batch must be >= 0, got %d", a->batch);
  if (a->vocab < 1 || a->vocab > kMaxVocab)
    return fail(VSAMP_E_ARG, "vocab must be in [1, %lld], got %d", static_cast<long long>(kMaxVocab),
                a->vocab);
  if (a->row_stride < a->vocab)
    return fail(VSAMP_E_ARG, "row_stride (%lld) must be >= vocab (%d)",
                static_cast<long long>(a->row_stride), a->vocab);
  if (a->batch > 0 && !a->logits) return fail(VSAMP_E_ARG, "logits is NULL");
  if ((a->hist_ids == nullptr) != (a->hist_offsets == nullptr) && a->hist_total > 0)
    return fail(VSAMP_E_ARG, "hist_ids and hist_offsets must both be set or both NULL");
  if (a->hist_total < 0 || a->hist_total >= (int64_t(1) << 31))
    return fail(VSAMP_E_ARG, "hist_total must be in [0, 2^31), got %lld",
                static_cast<long long>(a->hist_total));
  if (need_draw) {
    if (a->batch > 0 && !a->out_ids) return fail(VSAMP_E_ARG, "out_ids is NULL");
    if (a->batch > 0 && !a->uniforms) return fail(VSAMP_E_ARG, "uniforms is NULL");
    if ((a->draft_ids == nullptr) != (a->out_draft_prob == nullptr))
      return fail(VSAMP_E_ARG, "draft_ids and out_draft_prob must both be set or both NULL");
  }
  return VSAMP_OK;
}

bool wants_penalties(const vsamp_args* a) {
  return a->hist_ids && a->hist_offsets && a->hist_total > 0 &&
         (a->repetition_penalty || a->presence_penalty || a->frequency_penalty);
}

int check_workspace(const vsamp_args* a, const Layout& L) {
  if (a->workspace_bytes < L.total || (L.total && !a->workspace))
    return fail(VSAMP_E_WORKSPACE, "workspace of %zu bytes given, %zu needed", a->workspace_bytes, L.total);
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255u)
    return fail(VSAMP_E_WORKSPACE, "workspace must be 256-byte aligned");
  return VSAMP_OK;
}

vs::Workspace workspace_of(const vsamp_args* a, const Layout& L) {
  char* w = static_cast<char*>(a->workspace);
  vs::Workspace ws;
  ws.n_exc = reinterpret_cast<uint32_t*>(w + L.n_exc);
  ws.exc_id = reinterpret_cast<int32_t*>(w + L.exc_id);
  ws.exc_val = reinterpret_cast<float*>(w + L.exc_val);
  ws.exc_cnt = reinterpret_cast<int32_t*>(w + L.exc_cnt);
  return ws;
}

vs::PenaltyArgs penalty_args(const vsamp_args* a, const vs::Workspace& ws) {
  vs::PenaltyArgs p;
  p.logits = a->logits;
  p.stride = a->row_stride;
  p.V = a->vocab;
  p.rep = a->repetition_penalty;
  p.pres = a->presence_penalty;
  p.freq = a->frequency_penalty;
  p.hist = a->hist_ids;
  p.off = a->hist_offsets;
  p.hstep = (a->flags & VSAMP_HIST_RANGES) ? 2 : 1;
  p.ws = ws;
  p.dense_counts = nullptr;
  p.counts_stride = 0;
  return p;
}

template <class Tin>
int launch_penalties(const vs::PenaltyArgs& p, int B, hipStream_t st) {
  hipLaunchKernelGGL(vs::k_penalty_prep<Tin>, dim3(B), dim3(vs::kThreads), 0, st, p);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_penalty_prep");
}

template <class Tin>
int run_sample(const vsamp_args* a, float* probs, int64_t probs_stride, hipStream_t st,
               vs::RowState* state = nullptr, int param_div = 1, const float* tile_max = nullptr,
               uint32_t* tile_arrive = nullptr, int tile_G = 1) {
  const bool pen = wants_penalties(a);
  if (state && pen) return fail(VSAMP_E_ARG, "row states are written without penalties only");
  if ((a->flags & VSAMP_HIST_APPEND) && (state || probs))
    return fail(VSAMP_E_ARG, "VSAMP_HIST_APPEND goes with a call that draws from penalised rows");
  vs::SampleArgs s;
  std::memset(&s, 0, sizeof s);
  if (pen) {
    const Layout L = layout(a->batch, a->vocab, a->hist_total);
    if (int rc = check_workspace(a, L)) return rc;
    s.ws = workspace_of(a, L);
    s.pen = penalty_args(a, s.ws);
    s.has_exc = 1;
    s.off = a->hist_offsets;
    // (the drawn id goes behind each row's range: the caller's history buffer is writable)
    if (a->flags & VSAMP_HIST_APPEND) s.hist_out = const_cast<int32_t*>(a->hist_ids);
  }
  s.logits = a->logits;
  s.stride = a->row_stride;
  s.V = a->vocab;
  s.temp = a->temperature;
  s.topk = a->top_k;
  s.topp = a->top_p;
  s.minp = a->min_p;
  s.u = a->uniforms;
  s.draft = a->draft_ids;
  s.out_ids = a->out_ids;
  s.out_dprob = a->out_draft_prob;
  s.out_probs = probs;
  s.probs_stride = probs_stride;
  s.out_state = state;
  s.param_div = param_div;
  s.nrows = a->batch;
  if (tile_max) {  // (bf16 rows with the LM head's tile maxima: no split rows, no states)
    s.tile_max = tile_max;
    s.nT = (a->vocab + VSAMP_LM_TILE - 1) / VSAMP_LM_TILE;
    s.tile_arrive = tile_arrive;  // (set: tile_G workgroups per row compute the maxima first)
    s.tile_G = tile_G;
    const dim3 grid(a->batch * (tile_arrive ? tile_G : 1));
    if (pen)
      hipLaunchKernelGGL((vs::k_sample<Tin, true, false, false, true>), grid, dim3(vs::kThreads), 0, st, s);
    else
      hipLaunchKernelGGL((vs::k_sample<Tin, false, false, false, true>), grid, dim3(vs::kThreads), 0, st, s);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_sample (tile maxima)");
  }
  // Small batches of bf16 rows, when asked for: split rows if the workspace holds the records.
  const int G = (a->flags & VSAMP_SPLIT_ROWS) ? split_slices(a->batch, a->vocab) : 1;
  if (sizeof(Tin) == 2 && !state && !probs && G >= 2 && a->workspace &&
      !(reinterpret_cast<uintptr_t>(a->workspace) & 255u) &&
      a->workspace_bytes >= split_total(a->batch, a->vocab, a->hist_total) &&
      !(reinterpret_cast<uintptr_t>(a->logits) & 15u) && a->row_stride % vs::kBlk == 0) {
    uint8_t* rec = static_cast<uint8_t*>(a->workspace) + split_records(a->batch, a->vocab, a->hist_total);
    s.slices = rec;
    s.arrive = reinterpret_cast<vs::u64*>(rec + static_cast<size_t>(a->batch) * G * vs::kSliceRecord);
    s.epoch = next_epoch();
    s.G = G;
    if (pen)
      hipLaunchKernelGGL((vs::k_sample<Tin, true, false, true>), dim3(a->batch * G), dim3(vs::kThreads), 0, st, s);
    else
      hipLaunchKernelGGL((vs::k_sample<Tin, false, false, true>), dim3(a->batch * G), dim3(vs::kThreads), 0, st, s);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_sample (split rows)");
  }
  // One launch per step: the penalty phase runs at the start of the same kernel.
  if (state)  // (the verify's launches, which apply no penalties)
    hipLaunchKernelGGL((vs::k_sample<Tin, false, true>), dim3(a->batch), dim3(vs::kThreads), 0, st, s);
  else if (pen)
    hipLaunchKernelGGL((vs::k_sample<Tin, true>), dim3(a->batch), dim3(vs::kThreads), 0, st, s);
  else
    hipLaunchKernelGGL((vs::k_sample<Tin, false>), dim3(a->batch), dim3(vs::kThreads), 0, st, s);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_sample");
}

template <class Tin>
int run_tile_pass(const vsamp_args* a, float* tile_max, uint32_t* arrive, hipStream_t st) {
  const int nT = (a->vocab + VSAMP_LM_TILE - 1) / VSAMP_LM_TILE;
  // One launch while the rows' workgroups fit one round on the CUs: G per row, each the maxima of
  // at most 64 tiles (one or two 16-byte loads per thread), the last of a row's G finishing it;
  // larger batches take a launch of the maxima first (256-thread workgroups), then the draw.
  const int G = (nT + vs::kTileSharePasses * vs::kWave - 1) / (vs::kTileSharePasses * vs::kWave);
  if (static_cast<int64_t>(a->batch) * G <= vs::kTileFusedWorkgroups)
    return run_sample<Tin>(a, nullptr, 0, st, nullptr, 1, tile_max, arrive, G);
  hipLaunchKernelGGL(vs::k_tile_max<Tin>, dim3((nT + vs::kTilesPerBlock - 1) / vs::kTilesPerBlock, a->batch),
                     dim3(vs::kTileMaxThreads), 0, st, static_cast<const Tin*>(a->logits), a->row_stride, a->vocab, nT,
                     tile_max);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "launch k_tile_max");
  return run_sample<Tin>(a, nullptr, 0, st, nullptr, 1, tile_max);
}

struct VerifyLayout {
  size_t tids, dids, ts, ds, jr, done, sums, rej, nrej, total;
};

VerifyLayout verify_layout(int64_t B, int64_t K) {
  VerifyLayout L;
  const size_t nt = static_cast<size_t>(B * (K + 1)), nd = static_cast<size_t>(B * K);
  size_t o = 0;
  L.tids = o;
  o = align_up(o + 4 * nt);
  L.dids = o;
  o = align_up(o + 4 * nd);
  L.ts = o;
  o = align_up(o + sizeof(vs::RowState) * nt);
  L.ds = o;
  o = align_up(o + sizeof(vs::RowState) * nd);
  L.jr = o;
  o = align_up(o + 4 * static_cast<size_t>(B));
  L.done = o;
  o = align_up(o + 4 * static_cast<size_t>(B));
  L.sums = o;
  o = align_up(o + 8 * static_cast<size_t>(B) * vs::kMaxStripes);
  L.rej = o;
  o = align_up(o + 4 * static_cast<size_t>(B));
  L.nrej = o;
  o = align_up(o + 4);
  L.total = o;
  return L;
}

}  // namespace

extern "C" {

int vsamp_abi_version(void) { return VSAMP_ABI_VERSION; }

int vsamp_query(int device, char* why, size_t n) {
  if (why && n) why[0] = '\0';
  return check_device(device, why, n);
}

size_t vsamp_workspace_bytes(int32_t batch, int32_t vocab, int64_t hist_total) {
  if (batch < 0 || vocab < 1 || hist_total < 0) return 0;
  return layout(batch, vocab, hist_total).total;
}

size_t vsamp_split_workspace_bytes(int32_t batch, int32_t vocab, int64_t hist_total) {
  if (batch < 0 || vocab < 1 || hist_total < 0) return 0;
  return split_total(batch, vocab, hist_total);
}

int vsamp_sample(const vsamp_args* a, void* stream) {
  g_err.clear();
  if (int rc = validate(a, true)) return rc;
  if (a->batch == 0) return VSAMP_OK;
  if (int rc = check_current_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return a->dtype == VSAMP_BF16 ? run_sample<uint16_t>(a, nullptr, 0, st)
                                : run_sample<float>(a, nullptr, 0, st);
}

int vsamp_sample_tiles(const vsamp_args* a, const float* tile_max, void* stream) {
  g_err.clear();
  if (int rc = validate(a, true)) return rc;
  if (a->dtype != VSAMP_BF16) return fail(VSAMP_E_DTYPE, "vsamp_sample_tiles takes the bf16 logits of vsamp_lm_head");
  if (a->batch == 0) return VSAMP_OK;
  if (!tile_max) return fail(VSAMP_E_ARG, "tile_max is NULL");
  if (int rc = check_current_device()) return rc;
  return run_sample<uint16_t>(a, nullptr, 0, static_cast<hipStream_t>(stream), nullptr, 1, tile_max);
}

int vsamp_sample_tile_pass(const vsamp_args* a, float* tile_max, uint32_t* arrive, void* stream) {
  g_err.clear();
  if (int rc = validate(a, true)) return rc;
  if (a->batch == 0) return VSAMP_OK;
  if (!tile_max || !arrive) return fail(VSAMP_E_ARG, "tile_max and arrive must be set");
  if ((reinterpret_cast<uintptr_t>(tile_max) | reinterpret_cast<uintptr_t>(arrive)) & 3u)
    return fail(VSAMP_E_ARG, "tile_max and arrive must be 4-byte aligned");
  if (int rc = check_current_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return a->dtype == VSAMP_BF16 ? run_tile_pass<uint16_t>(a, tile_max, arrive, st)
                                : run_tile_pass<float>(a, tile_max, arrive, st);
}

int vsamp_sample_noalloc(const vsamp_args* a, void* stream) {
  g_err.clear();
  if (int rc = validate(a, true)) return rc;
  if (a->workspace || a->workspace_bytes)
    return fail(VSAMP_E_ARG, "vsamp_sample_noalloc uses the library's own workspace: leave workspace NULL");
  if (a->batch == 0) return VSAMP_OK;
  if (int rc = check_current_device()) return rc;
  const size_t need = layout(a->batch, a->vocab, a->hist_total).total;
  if (wants_penalties(a) && need > kScratchBytes)
    return fail(VSAMP_E_WORKSPACE,
                "vsamp_sample_noalloc: batch %d with %lld history ids needs %zu workspace bytes, more than its "
                "%zu; use vsamp_sample with a caller workspace",
                a->batch, static_cast<long long>(a->hist_total), need, kScratchBytes);
  vsamp_args c = *a;  // (the slice records of split rows too, when they fit)
  if (int rc = scratch_of_current_device(&c.workspace)) return rc;
  c.workspace_bytes = kScratchBytes;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return c.dtype == VSAMP_BF16 ? run_sample<uint16_t>(&c, nullptr, 0, st) : run_sample<float>(&c, nullptr, 0, st);
}

int vsamp_probs(const vsamp_args* a, float* out, int64_t out_stride, void* stream) {
  g_err.clear();
  if (int rc = validate(a, false)) return rc;
  if (a->batch == 0) return VSAMP_OK;
  if (!out) return fail(VSAMP_E_ARG, "out is NULL");
  if (out_stride < a->vocab) return fail(VSAMP_E_ARG, "out_stride must be >= vocab");
  if (int rc = check_current_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return a->dtype == VSAMP_BF16 ? run_sample<uint16_t>(a, out, out_stride, st)
                                : run_sample<float>(a, out, out_stride, st);
}

int vsamp_penalized_logits(const vsamp_args* a, float* out, int32_t* counts, int64_t out_stride,
                           void* stream) {
  g_err.clear();
  if (int rc = validate(a, false)) return rc;
  if (a->batch == 0) return VSAMP_OK;
  if (!out) return fail(VSAMP_E_ARG, "out is NULL");
  if (out_stride < a->vocab) return fail(VSAMP_E_ARG, "out_stride must be >= vocab");
  if (int rc = check_current_device()) return rc;
  const Layout L = layout(a->batch, a->vocab, a->hist_total);
  if (int rc = check_workspace(a, L)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  vs::PenaltyArgs p = penalty_args(a, workspace_of(a, L));
  if (!wants_penalties(a)) {
    p.rep = p.pres = p.freq = nullptr;  // every row off: exceptions stay empty
  }
  if (!(a->hist_ids && a->hist_offsets)) {
    p.hist = nullptr;
    p.off = nullptr;
  }
  p.dense_counts = counts;
  p.counts_stride = out_stride;
  int rc = a->dtype == VSAMP_BF16 ? launch_penalties<uint16_t>(p, a->batch, st)
                                  : launch_penalties<float>(p, a->batch, st);
  if (rc) return rc;
  if (a->dtype == VSAMP_BF16)
    hipLaunchKernelGGL(vs::k_penalized_out<uint16_t>, dim3(a->batch), dim3(vs::kThreads), 0, st, p, out,
                       out_stride);
  else
    hipLaunchKernelGGL(vs::k_penalized_out<float>, dim3(a->batch), dim3(vs::kThreads), 0, st, p, out,
                       out_stride);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_penalized_out");
}

size_t vsamp_verify_workspace_bytes(int32_t batch, int32_t num_draft) {
  if (batch < 0 || num_draft < 1) return 0;
  return verify_layout(batch, num_draft).total;
}

int vsamp_verify(const vsamp_verify_args* v, void* stream) {
  g_err.clear();
  if (!v) return fail(VSAMP_E_ARG, "args is NULL");
  const int B = v->batch, K = v->num_draft;
  if (B < 0) return fail(VSAMP_E_ARG, "batch must be >= 0, got %d", B);
  if (K < 1 || K > 64) return fail(VSAMP_E_ARG, "num_draft must be in [1, 64], got %d", K);
  vsamp_args t = v->target, d = v->draft;
  if (t.batch != B * (K + 1))
    return fail(VSAMP_E_ARG, "target.batch must be batch * (num_draft + 1) = %d, got %d", B * (K + 1), t.batch);
  if (d.batch != B * K)
    return fail(VSAMP_E_ARG, "draft.batch must be batch * num_draft = %d, got %d", B * K, d.batch);
  if (t.vocab != d.vocab) return fail(VSAMP_E_ARG, "target and draft vocab differ (%d, %d)", t.vocab, d.vocab);
  if (t.dtype != d.dtype) return fail(VSAMP_E_DTYPE, "target and draft logits dtypes differ");
  if (t.draft_ids || t.out_ids || t.out_draft_prob || d.draft_ids || d.out_ids || d.out_draft_prob)
    return fail(VSAMP_E_ARG, "draft_ids and outputs of target and draft are set by the call: leave them NULL");
  if (wants_penalties(&t) || wants_penalties(&d))
    return fail(VSAMP_E_ARG, "verify does not apply penalties (histories must be NULL)");
  if (B > 0 && (!v->draft_tokens || !v->u_accept || !v->u_residual || !v->out_tokens || !v->out_count))
    return fail(VSAMP_E_ARG, "draft_tokens, u_accept, u_residual, out_tokens and out_count must be set");
  if (!d.uniforms) d.uniforms = v->u_residual;  // (the draft rows' own draws are not used)
  const VerifyLayout L = verify_layout(B, K);
  if (v->workspace_bytes < L.total || (L.total && !v->workspace))
    return fail(VSAMP_E_WORKSPACE, "workspace of %zu bytes given, %zu needed", v->workspace_bytes, L.total);
  if (reinterpret_cast<uintptr_t>(v->workspace) & 255u)
    return fail(VSAMP_E_WORKSPACE, "workspace must be 256-byte aligned");
  char* w = static_cast<char*>(v->workspace);
  int32_t* tids = reinterpret_cast<int32_t*>(w + L.tids);
  int32_t* dids = reinterpret_cast<int32_t*>(w + L.dids);
  vs::RowState* ts = reinterpret_cast<vs::RowState*>(w + L.ts);
  vs::RowState* ds = reinterpret_cast<vs::RowState*>(w + L.ds);
  t.out_ids = tids;
  d.out_ids = dids;  // (the draft rows' own draws are not used)
  if (int rc = validate(&t, true)) return rc;
  if (int rc = validate(&d, true)) return rc;
  if (B == 0) return VSAMP_OK;
  if (int rc = check_current_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf = t.dtype == VSAMP_BF16;
  // parameters and uniforms: one entry per sequence for all of its rows
  if (int rc = bf ? run_sample<uint16_t>(&t, nullptr, 0, st, ts, K + 1) : run_sample<float>(&t, nullptr, 0, st, ts, K + 1))
    return rc;
  if (v->draft_states) {
    if (reinterpret_cast<uintptr_t>(v->draft_states) & 7u) return fail(VSAMP_E_ARG, "draft_states must be 8-byte aligned");
    ds = static_cast<vs::RowState*>(const_cast<void*>(v->draft_states));
  } else if (int rc = bf ? run_sample<uint16_t>(&d, nullptr, 0, st, ds, K) : run_sample<float>(&d, nullptr, 0, st, ds, K)) {
    return rc;
  }
  vs::VerifyArgs a;
  a.tgt = t.logits;
  a.tstride = t.row_stride;
  a.drf = d.logits;
  a.dstride = d.row_stride;
  a.V = t.vocab;
  a.K = K;
  a.drafts = v->draft_tokens;
  a.u_acc = v->u_accept;
  a.u_res = v->u_residual;
  a.tids = tids;
  a.ts = ts;
  a.ds = ds;
  a.out_tokens = v->out_tokens;
  a.out_count = v->out_count;
  a.jr = reinterpret_cast<int32_t*>(w + L.jr);
  a.done = reinterpret_cast<uint32_t*>(w + L.done);
  a.sums = reinterpret_cast<vs::u64*>(w + L.sums);
  a.rej = reinterpret_cast<int32_t*>(w + L.rej);
  a.nrej = reinterpret_cast<int32_t*>(w + L.nrej);
  const int nstripes = ((t.vocab + vs::kBlk - 1) / vs::kBlk + vs::kThreads - 1) / vs::kThreads;
  a.max_slices = 1;
  while (2 * a.max_slices <= nstripes && 2 * a.max_slices <= kMaxResidualSlices) a.max_slices *= 2;
  // at most one workgroup per CU: items beyond the rejected rows' exit without holding a CU
  const int64_t items = B * a.max_slices;
  const dim3 gr(static_cast<unsigned>(items < current_cus() ? items : current_cus()));
  if (bf) {
    hipLaunchKernelGGL(vs::k_verify_accept<uint16_t>, dim3(1), dim3(vs::kThreads), 0, st, a, B);
    hipLaunchKernelGGL(vs::k_verify_residual<uint16_t>, gr, dim3(vs::kThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL(vs::k_verify_accept<float>, dim3(1), dim3(vs::kThreads), 0, st, a, B);
    hipLaunchKernelGGL(vs::k_verify_residual<float>, gr, dim3(vs::kThreads), 0, st, a);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_verify");
}

int vsamp_logprobs(const vsamp_args* a, const int32_t* tokens, int32_t n_top, float* out_token_logprob,
                   int32_t* out_top_ids, float* out_top_logprobs, void* stream) {
  g_err.clear();
  if (!a) return fail(VSAMP_E_ARG, "args is NULL");
  if (a->dtype != VSAMP_BF16 && a->dtype != VSAMP_F32)
    return fail(VSAMP_E_DTYPE, "unsupported logits dtype %d (VSAMP_BF16=0, VSAMP_F32=1)", a->dtype);
  if (a->batch < 0) return fail(VSAMP_E_ARG, "batch must be >= 0, got %d", a->batch);
  if (a->vocab < 1 || a->vocab > kMaxVocab)
    return fail(VSAMP_E_ARG, "vocab must be in [1, %lld], got %d", static_cast<long long>(kMaxVocab), a->vocab);
  if (a->row_stride < a->vocab)
    return fail(VSAMP_E_ARG, "row_stride (%lld) must be >= vocab (%d)", static_cast<long long>(a->row_stride),
                a->vocab);
  if (n_top < 0 || n_top > vs::kMaxTop) return fail(VSAMP_E_ARG, "n_top must be in [0, %d], got %d", vs::kMaxTop, n_top);
  if ((tokens == nullptr) != (out_token_logprob == nullptr))
    return fail(VSAMP_E_ARG, "tokens and out_token_logprob must both be set or both NULL");
  if (n_top > 0 && (!out_top_ids || !out_top_logprobs))
    return fail(VSAMP_E_ARG, "out_top_ids and out_top_logprobs must be set when n_top > 0");
  if (a->batch == 0) return VSAMP_OK;
  if (!a->logits) return fail(VSAMP_E_ARG, "logits is NULL");
  if (int rc = check_current_device()) return rc;
  vs::LogprobArgs l;
  l.logits = a->logits;
  l.stride = a->row_stride;
  l.V = a->vocab;
  l.tokens = tokens;
  l.n_top = n_top;
  l.out_token = out_token_logprob;
  l.out_top_ids = out_top_ids;
  l.out_top = out_top_logprobs;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->dtype == VSAMP_BF16)
    hipLaunchKernelGGL(vs::k_logprobs<uint16_t>, dim3(a->batch), dim3(vs::kThreads), 0, st, l);
  else
    hipLaunchKernelGGL(vs::k_logprobs<float>, dim3(a->batch), dim3(vs::kThreads), 0, st, l);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_logprobs");
}

int vsamp_logprobs_tiles(const vsamp_args* a, const float* tile_max, const float* tile_sum, const int32_t* tokens,
                         int32_t n_top, float* out_token_logprob, int32_t* out_top_ids, float* out_top_logprobs,
                         void* stream) {
  g_err.clear();
  if (!a) return fail(VSAMP_E_ARG, "args is NULL");
  if (a->dtype != VSAMP_BF16) return fail(VSAMP_E_DTYPE, "vsamp_logprobs_tiles takes the bf16 logits of vsamp_lm_head");
  if (a->batch < 0) return fail(VSAMP_E_ARG, "batch must be >= 0, got %d", a->batch);
  if (a->vocab < 1 || a->vocab > kMaxVocab)
    return fail(VSAMP_E_ARG, "vocab must be in [1, %lld], got %d", static_cast<long long>(kMaxVocab), a->vocab);
  if (a->row_stride < a->vocab)
    return fail(VSAMP_E_ARG, "row_stride (%lld) must be >= vocab (%d)", static_cast<long long>(a->row_stride),
                a->vocab);
  if (n_top < 0 || n_top > vs::kMaxTop) return fail(VSAMP_E_ARG, "n_top must be in [0, %d], got %d", vs::kMaxTop, n_top);
  if ((tokens == nullptr) != (out_token_logprob == nullptr))
    return fail(VSAMP_E_ARG, "tokens and out_token_logprob must both be set or both NULL");
  if (n_top > 0 && (!out_top_ids || !out_top_logprobs))
    return fail(VSAMP_E_ARG, "out_top_ids and out_top_logprobs must be set when n_top > 0");
  if (a->batch == 0) return VSAMP_OK;
  if (!a->logits || !tile_max || !tile_sum) return fail(VSAMP_E_ARG, "logits, tile_max and tile_sum must be set");
  if (int rc = check_current_device()) return rc;
  vs::LogprobArgs l;
  l.logits = a->logits;
  l.stride = a->row_stride;
  l.V = a->vocab;
  l.tokens = tokens;
  l.n_top = n_top;
  l.out_token = out_token_logprob;
  l.out_top_ids = out_top_ids;
  l.out_top = out_top_logprobs;
  l.tmax = tile_max;
  l.tsum = tile_sum;
  l.nT = (a->vocab + VSAMP_LM_TILE - 1) / VSAMP_LM_TILE;
  hipLaunchKernelGGL((vs::k_logprobs<uint16_t, true>), dim3(a->batch), dim3(vs::kThreads), 0,
                     static_cast<hipStream_t>(stream), l);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_logprobs (tiles)");
}

int vsamp_lm_head(const vsamp_lm_head_args* a, void* stream) {
  g_err.clear();
  if (!a) return fail(VSAMP_E_ARG, "args is NULL");
  if (a->batch < 0) return fail(VSAMP_E_ARG, "batch must be >= 0, got %d", a->batch);
  if (a->vocab < 1 || a->vocab > kMaxVocab)
    return fail(VSAMP_E_ARG, "vocab must be in [1, %lld], got %d", static_cast<long long>(kMaxVocab), a->vocab);
  if (a->dim < vs::kLmBK || a->dim % vs::kLmBK)
    return fail(VSAMP_E_ARG, "dim must be a positive multiple of %d, got %d", vs::kLmBK, a->dim);
  if (a->hidden_stride < a->dim || a->weight_stride < a->dim || a->logits_stride < a->vocab)
    return fail(VSAMP_E_ARG, "strides must be >= dim (hidden, weight) and >= vocab (logits)");
  if (a->batch == 0) return VSAMP_OK;
  if (!a->hidden || !a->weight || !a->logits || !a->tile_max || !a->tile_sum)
    return fail(VSAMP_E_ARG, "hidden, weight, logits, tile_max and tile_sum must be set");
  if ((reinterpret_cast<uintptr_t>(a->hidden) | reinterpret_cast<uintptr_t>(a->weight)) & 15u ||
      a->hidden_stride % 8 || a->weight_stride % 8)
    return fail(VSAMP_E_ARG, "hidden and weight rows must be 16-byte aligned (aligned base, stride a multiple of 8)");
  if (int rc = check_current_device()) return rc;
  vs::LmHeadArgs l;
  l.hidden = static_cast<const uint16_t*>(a->hidden);
  l.ldh = a->hidden_stride;
  l.W = static_cast<const uint16_t*>(a->weight);
  l.ldw = a->weight_stride;
  l.logits = static_cast<uint16_t*>(a->logits);
  l.ldo = a->logits_stride;
  l.tmax = a->tile_max;
  l.tsum = a->tile_sum;
  l.nT = (a->vocab + VSAMP_LM_TILE - 1) / VSAMP_LM_TILE;
  l.B = a->batch;
  l.d = a->dim;
  l.V = a->vocab;
  l.vec_out = !(reinterpret_cast<uintptr_t>(a->logits) & 15u) && a->logits_stride % 8 == 0;
  static_assert(vs::kLmBN == VSAMP_LM_TILE, "the statistics' tile is the kernel's column tile");
  // (up to 4 rows: matrix-vector products, for the hidden sizes they are built for; batches of
  // at most 64 rows: the weight streamed into registers, 640 vocabulary rows a workgroup; larger
  // batches: 256 x 128 tiles with both operands staged through LDS)
  const int cpl = a->dim % 512 == 0 ? a->dim / 512 : 0;  // hidden chunks per lane
  if (a->batch <= 4 && (cpl == 1 || cpl == 2 || cpl == 4 || cpl == 8)) {
    const int nb = a->batch == 1 ? 1 : a->batch == 2 ? 2 : 4;
    const dim3 grid(l.nT), block(vs::kGvThreads);
    const hipStream_t st = static_cast<hipStream_t>(stream);
#define VS_GEMV(C, N) if (cpl == C && nb == N) hipLaunchKernelGGL((vs::k_lm_gemv<C, N>), grid, block, 0, st, l)
    VS_GEMV(1, 1); VS_GEMV(2, 1); VS_GEMV(4, 1); VS_GEMV(8, 1);
    VS_GEMV(1, 2); VS_GEMV(2, 2); VS_GEMV(4, 2); VS_GEMV(8, 2);
    VS_GEMV(1, 4); VS_GEMV(2, 4); VS_GEMV(4, 4); VS_GEMV(8, 4);
#undef VS_GEMV
  } else if (a->batch <= 64)
    hipLaunchKernelGGL(vs::k_lm_stream, dim3((a->vocab + vs::kLsRows - 1) / vs::kLsRows), dim3(vs::kLsThreads), 0,
                       static_cast<hipStream_t>(stream), l);
  else
    hipLaunchKernelGGL(vs::k_lm_head<256>, dim3(l.nT, (a->batch + 255) / 256), dim3(vs::kLmThreads), 0,
                       static_cast<hipStream_t>(stream), l);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_lm_head");
}

int vsamp_tile_stats(const void* logits, int64_t row_stride, int32_t batch, int32_t vocab, float* tile_max,
                     float* tile_sum, void* stream) {
  g_err.clear();
  if (batch < 0) return fail(VSAMP_E_ARG, "batch must be >= 0, got %d", batch);
  if (vocab < 1 || vocab > kMaxVocab)
    return fail(VSAMP_E_ARG, "vocab must be in [1, %lld], got %d", static_cast<long long>(kMaxVocab), vocab);
  if (row_stride < vocab)
    return fail(VSAMP_E_ARG, "row_stride (%lld) must be >= vocab (%d)", static_cast<long long>(row_stride), vocab);
  if (batch == 0) return VSAMP_OK;
  if (!logits || !tile_max || !tile_sum) return fail(VSAMP_E_ARG, "logits, tile_max and tile_sum must be set");
  if (int rc = check_current_device()) return rc;
  const int nT = (vocab + VSAMP_LM_TILE - 1) / VSAMP_LM_TILE;
  constexpr int kTiles = vs::kTsThreads / 16;
  hipLaunchKernelGGL(vs::k_tile_stats, dim3((nT + kTiles - 1) / kTiles, batch), dim3(vs::kTsThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(logits), row_stride, vocab, nT,
                     tile_max, tile_sum);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_tile_stats");
}

int vsamp_sample_states(const vsamp_args* a, void* out_states, void* stream) {
  g_err.clear();
  if (int rc = validate(a, true)) return rc;
  if (a->batch == 0) return VSAMP_OK;
  if (!out_states || (reinterpret_cast<uintptr_t>(out_states) & 7u))
    return fail(VSAMP_E_ARG, "out_states must be set and 8-byte aligned");
  if (wants_penalties(a)) return fail(VSAMP_E_ARG, "row states are written without penalties only");
  if (int rc = check_current_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  vs::RowState* s = static_cast<vs::RowState*>(out_states);
  return a->dtype == VSAMP_BF16 ? run_sample<uint16_t>(a, nullptr, 0, st, s) : run_sample<float>(a, nullptr, 0, st, s);
}

int vsamp_uniforms(const int64_t* seeds, const int64_t* positions, int32_t n, float* out) {
  g_err.clear();
  if (n < 0) return fail(VSAMP_E_ARG, "n must be >= 0, got %d", n);
  if (n > 0 && (!seeds || !positions || !out)) return fail(VSAMP_E_ARG, "seeds, positions and out must be set");
  for (int32_t i = 0; i < n; ++i) out[i] = vs_host::position_uniform(seeds[i], positions[i]);
  return VSAMP_OK;
}

int vsamp_uniforms_device(const int64_t* seeds, const int64_t* positions, int32_t n, float* out, void* stream) {
  g_err.clear();
  if (n < 0) return fail(VSAMP_E_ARG, "n must be >= 0, got %d", n);
  if (n == 0) return VSAMP_OK;
  if (!seeds || !positions || !out) return fail(VSAMP_E_ARG, "seeds, positions and out must be set");
  if (int rc = check_current_device()) return rc;
  hipLaunchKernelGGL(vs_host::k_uniforms, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     seeds, positions, static_cast<int>(n), out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_uniforms");
}

int vsamp_spec_advance(int64_t* inputs, int32_t n, int32_t num_draft, const int32_t* tokens, const int32_t* counts,
                       const int64_t* seeds, float* uniforms, void* stream) {
  g_err.clear();
  if (n < 0) return fail(VSAMP_E_ARG, "n must be >= 0, got %d", n);
  if (num_draft < 1 || 3 * num_draft + 1 > 64) return fail(VSAMP_E_ARG, "num_draft must be in [1, 21], got %d", num_draft);
  if (n == 0) return VSAMP_OK;
  if (!inputs || !seeds || !uniforms) return fail(VSAMP_E_ARG, "inputs, seeds and uniforms must be set");
  if (!tokens != !counts) return fail(VSAMP_E_ARG, "tokens and counts are given together or not at all");
  if (int rc = check_current_device()) return rc;
  int G = 1;
  while (G < 3 * num_draft + 1) G *= 2;
  hipLaunchKernelGGL(vs_host::k_spec_advance, dim3((n * G + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     inputs, static_cast<int>(n), static_cast<int>(num_draft), G, tokens, counts, seeds, uniforms);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VSAMP_OK : hip_fail(e, "launch k_spec_advance");
}

const char* vsamp_last_error(void) { return g_err.c_str(); }

}  // extern "C"
