// Per-row sampling kernel: one 1024-thread workgroup per row.
//
// Everything is decided on penalised fp32 logits x. Temperature scaling z = fl32(x / T) is
// monotone non-decreasing in x, so every filter is a threshold on x:
//   top-k  : the kth largest x (exact order statistic), then the smallest x whose z reaches
//            z(kth) (bisection over keys, which also covers division merging distinct x)
//   min-p  : the smallest x with exp(z - max z) >= min_p (fp64), by bisection over keys
//   top-p  : the cutoff value (the lowest value whose mass strictly above it is < P), and how
//            many of its tokens are kept, in ascending id order
//   draw   : the value group where the descending cumulative mass crosses u * S, and the
//            member of that group (ascending id) it lands on
// Masses are q = rint(p~ * 2^42) with p~ = exp(z - max z) in fp64, summed as integers: exact
// and order-independent.
//
// bf16 rows (fast path): one pass builds a histogram of the row's 65536 possible 16-bit keys
// (u16 counts packed in pairs, 128 KB of LDS) while it counts the row's token history in an LDS
// hash table. Every threshold and the draw's value group are then found from the histogram:
// per-chunk (64-key) counts and masses computed by all waves, and the decisions (totals, top-k,
// min-p, top-p, the draw) taken by wave 0 alone from a scan over chunks and a walk inside one
// chunk, with fp64 exps only for populated keys. A second, compare-only pass over the blocks
// of the threads that can hold the drawn value finds the id of the drawn token. fp32 rows, and
// bf16 rows whose histogram or history table cannot hold them, take the generic path: a
// workspace penalty pass, then radix descents over 32-bit ordered keys.
//
// Penalised tokens ("exceptions"): the generic path masks them out of logits reads by the row's
// bitmap and visits them from the workspace's list; the fast path keeps the list in LDS and
// takes their original keys back out of the histogram.
#pragma once

#include "common.cuh"
#include "penalty.cuh"
#include "split.cuh"

namespace vs {

// A row's kept set and normalisation as the sampling kernel found them: with it a later kernel
// recomputes any token's final probability, bit for bit as probs mode writes it.
struct RowState {
  float mz, T, x0, vc;           // max scaled logit, temperature, cutoff value, cutoff group value
  int32_t partial, idr, point;   // the cutoff group split at id idr; a point mass at `point`
  int32_t pad;
  u64 S;                         // kept mass (fixed point, 2^42)
};
static_assert(sizeof(RowState) == 40, "VSAMP_ROW_STATE_BYTES");

struct SampleArgs {
  const void* logits;
  int64_t stride;
  int V;
  const float* temp;
  const int32_t* topk;
  const float* topp;
  const float* minp;
  const float* u;
  const int32_t* draft;
  int32_t* out_ids;
  int32_t* hist_out;  // when non-null, each row's drawn id also goes to hist_out[its history's end]
  float* out_dprob;
  float* out_probs;  // probs mode when non-null
  int64_t probs_stride;
  RowState* out_state;  // optional: each row's RowState
  int param_div;        // (row-state launches) rows per parameter entry: row r reads entry r / param_div
  Workspace ws;
  int has_exc;  // the workspace holds this batch's exceptions
  const int32_t* off;
  PenaltyArgs pen;  // the penalty phase's inputs (used when the kernel runs it)
  // split rows (G > 1): workgroup b takes slice b / nrows of row b % nrows
  uint8_t* slices;  // the rows' slice records, G per row
  u64* arrive;      // per row: (epoch << 16 | slices arrived)
  u64 epoch;        // this launch's tag (48 bits), distinct from every earlier launch's
  int G;            // slices per row (0: one workgroup per row)
  int nrows;        // B
  // (vsamp_sample_tiles) the rows' tile maxima [B, nT], one per kStatTile logits
  const float* tile_max;
  int nT;
  // (vsamp_sample_tile_pass, one launch) tile_G workgroups per row compute the maxima, and the
  // last to count itself in at the row's arrival word (zero between launches) finishes the row
  uint32_t* tile_arrive;
  int tile_G;
};

// The row of this workgroup.
__device__ __forceinline__ int row_index(const SampleArgs& a) {
  return a.G > 1 ? static_cast<int>(blockIdx.x % static_cast<unsigned>(a.nrows)) : static_cast<int>(blockIdx.x);
}

// Scratch of the id-order search.
struct Search {
  float vslot;
  u64 red64[kWaves];
  u64 cell[kWaves][kMaxStripes];
  u64 tw[kThreads];
  u64 slot[kBlk];
  uint32_t slot_mask;
  int bi[4];
  u64 bq[4];
};

// Scratch of the generic path's radix descents.
struct Radix {
  uint32_t hcnt[256];
  u64 hmass[256];
  uint32_t bk[4];
  u64 bq[4];
  uint32_t ncand;  // elements >= x0 (the candidate list's length when it fits)
};

// The generic path's candidates: the elements >= x0 (bulk values and penalised values), copied
// to LDS when at most kCandCap of them, so that the top-p cutoff and the draw descend over the
// list instead of re-reading the row (two 4-level descents: eight passes over the row).
struct Cand {
  float x;
  int32_t id;
};
constexpr int kCandCap = 4096;
struct CandList {
  const Cand* c;
  int n;
};

struct GenericSmem {
  Search srch;
  Radix rdx;
};

// After the histogram (or on the generic path) the 128 KB buffer holds, in words:
//   [0, kBitmapOffset)                          Search and Radix scratch
//   [kBitmapOffset, kBitmapOffset + 16384)      per-block lane masks of penalised ids (V / 8 bytes)
//   [kMatchOffset, kMatchOffset + kMatchWords)  the draw's per-block count cells
constexpr int kBitmapOffset = kPenBitmapOffset;  // (where the penalty pass's bitmap path leaves its bitmap)
constexpr int kMatchOffset = kBitmapOffset + 16384;

constexpr int kMaxL = 128;     // penalised values in one chunk the fast path can resolve
constexpr int kExcCap = 2048;  // penalised ids per row the fast path keeps in LDS
constexpr int kMatchWords = 8192;  // LDS words of the draw's per-block count cells (V <= 262144)

// A row's parameters, as 32-bit words in this order (absent columns take the defaults below).
struct RowParams {
  float T, tp, mp, u;
  int K, draft;
  float rep, pres, freq;  // penalties
  int h0, h1;             // the row's history: hist_ids[h0, h1)
};
constexpr int kParamWords = 11;
static_assert(sizeof(RowParams) == 4 * kParamWords, "RowParams is 32-bit words");

// What wave 0 decides between the fast path's parallel phases (one LDS copy, read by all).
struct FastPlan {
  int status;  // kPlanFast, kPlanGeneric or kPlanPoint
  uint32_t mkey, nnan;
  float x0, mz;
  // the kept set (Kept's fields) and the draw
  float vc, vd;
  int partial, has_cut;
  uint32_t r;
  u64 mabove_c, qc, S, j;
};
constexpr int kPlanFast = 0, kPlanGeneric = 1, kPlanPoint = 2;

struct __align__(16) FastSmem {
  // ccnt, cmass and eval also hold the history's hash table while the row's histogram is built
  uint32_t ccnt[kThreads];  // per-chunk element counts
  u64 cmass[kThreads];      // per-chunk masses of elements >= x0
  float eval[kExcCap];      // the row's penalised values and ids (in no particular order)
  int32_t eid[kExcCap];
  uint32_t lkey[kMaxL];     // one chunk's penalised values: ordered key
  u64 lq[kMaxL];            //   and mass
  uint32_t binc[kWave];     // per-key counts / masses of penalised values inside that chunk
  u64 binm[kWave];
  uint32_t pchunk[2];  // the chunks that hold penalised values lie in [pchunk[0], pchunk[1]]
  uint32_t red32[kWaves];
  u64 red64[2 * kWaves];
  uint32_t sk[8];
  u64 sq[8];
  int si[8];
  uint32_t hfail;  // the history's hash table overflowed a probe sequence
  RowParams prm;   // this row's parameters
  uint4 wp[kWaves];  // per-wave partials: count, NaNs, top chunk code, penalised max key
  FastPlan plan;
};


// 16-byte block b of a bf16 row.
__device__ __align__(16) uint16_t g_unused_block[kBlk];  // (read, never written)

__device__ __forceinline__ uint4 ld_block(const uint16_t* base, int b) {
  const u32x4_t v = ld_global(reinterpret_cast<const u32x4_t*>(base + b * kBlk));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// defaults of the parameter words (RowParams order): T 1, top-p 1, min-p 0, u 0, top-k 0,
// draft -1, repetition 1, presence 0, frequency 0, history [0, 0)
__device__ const uint32_t kParamDefaults[16] = {0x3F800000u, 0x3F800000u, 0u, 0u, 0u, 0xFFFFFFFFu, 0x3F800000u,
                                                0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};

// Parameter word w of row r (w >= kParamWords: a default, unused): every column is loaded
// (uniform addresses, one load each) and the lane picks its word; selecting the column per lane
// instead would index the argument struct, which then has to live in scratch memory.
// Word w of row r's parameters, one load per lane: the lane picks its column's address (or the
// default's) first, so nothing waits for the load until the word is used.
template <bool PEN, bool STATE = false>
__device__ __forceinline__ uint32_t param_word(const SampleArgs& a, int r0, int w) {
  const int r = STATE ? r0 / a.param_div : r0;
  const void* cols[kParamWords] = {a.temp, a.topp, a.minp, a.u, a.topk, a.draft,
                                   PEN ? a.pen.rep : nullptr, PEN ? a.pen.pres : nullptr,
                                   PEN ? a.pen.freq : nullptr, PEN ? a.off : nullptr, PEN ? a.off : nullptr};
  const void* c = nullptr;
#pragma unroll
  for (int k = 0; k < kParamWords; ++k) c = w == k ? cols[k] : c;
  const int i = w >= kParamWords - 2 ? r * (PEN ? a.pen.hstep : 1) + (w - (kParamWords - 2)) : r;
  const uint32_t* q = c ? static_cast<const uint32_t*>(c) + i : &kParamDefaults[w];
  return ld_global(q);
}

// floor(n / d), d > 0, for quotients below 2^32 (a member index): the double quotient is within
// one of it (each operand and the division round by at most 2^-53), so one step up or down in
// integers makes it exact -- a fraction of the 64-bit integer division's instructions.
__device__ __forceinline__ u64 div_index(u64 n, u64 d) {
  u64 q = static_cast<u64>(static_cast<double>(n) / static_cast<double>(d));
  if (q * d > n) --q;
  else if (n - q * d >= d) ++q;
  return q;
}

// ---- the fast path's history count ----------------------------------------------------------
// A history of at most kFastMaxL ids is counted in a kFastSlots-word LDS hash table over
// ccnt/cmass/eval (dead until the histogram is complete) whose words pack (id << 13 | count):
// ids are below 2^19 and counts below 8191, so a word is never kEmpty. Linear probing; a probe
// sequence longer than kFastProbes sends the row to the generic path.
constexpr int kFastSlots = 4096;
constexpr int kFastHistPer = 8;  // history ids per thread
constexpr int kFastMaxL = kFastHistPer * kThreads - 2;
constexpr int kFastProbes = 64;
static_assert(offsetof(FastSmem, cmass) == sizeof(uint32_t) * kThreads &&
                  offsetof(FastSmem, eval) == offsetof(FastSmem, cmass) + sizeof(u64) * kThreads &&
                  offsetof(FastSmem, eval) + sizeof(float) * kExcCap >= sizeof(uint32_t) * kFastSlots,
              "the hash table must fit over ccnt, cmass and eval");
static_assert(kMaxStripes * kThreads * kBlk <= (1 << 19) && kFastMaxL < 8191, "hash word fields");

__device__ __forceinline__ uint32_t* fast_htab(FastSmem& f) { return f.ccnt; }

// Counts one occurrence of `id`; false if its probe sequence found neither it nor a free slot.
__device__ __forceinline__ bool fast_insert(uint32_t* htab, uint32_t id) {
  uint32_t h = (id * 2654435761u) >> (32 - 12);  // Fibonacci hashing onto 4096 slots
  const uint32_t tag = id << 13;
  for (int n = 0; n < kFastProbes; ++n) {
    const uint32_t prev = atomicCAS(&htab[h], kEmpty, tag | 1u);
    if (prev == kEmpty) return true;
    if ((prev & 0xFFFFE000u) == tag) {
      atomicAdd(&htab[h], 1u);
      return true;
    }
    h = (h + 1) & (kFastSlots - 1);
  }
  return false;
}

// Up to kPresMaxV ids the history is counted without hashing, in the same LDS (words of
// ccnt .. eid, in order): a presence bitmap of the vocabulary (one bit per id, 64-bit words
// from word kPresBits), the exclusive prefix of the bitmap words' popcounts (u16, after the
// bitmap) and u16 counts indexed by the rank of an id among the distinct ids (words 0 ..
// kThreads - 1). Setting the bits takes one non-returning atomic per id; ranks come from the
// prefix and a popcount; a rank's id is written by the thread that owns its bitmap word (words
// kPresPer * t .. + kPresPer - 1 belong to thread t) into words kPresBits .. (over the dead
// bitmap). Distinct ids end in ascending id order.
constexpr int kPresBits = kThreads;  // first word of the bitmap (and of the ids in rank order)
constexpr int kPresRegion = kThreads + 2 * kThreads + 2 * kExcCap;  // words of ccnt .. eid
constexpr int kPresPer = 3;          // bitmap words per thread
constexpr int kPresMaxWords = (2 * (kPresRegion - kPresBits)) / 5;  // 64-bit words: 2 + 1/2 u32 each
constexpr int kPresMaxV = 64 * kPresMaxWords;
static_assert(kPresMaxWords <= kPresPer * kThreads && kPresBits + kExcCap <= offsetof(FastSmem, eval) / 4,
              "bitmap words per thread; the ids in rank order must lie below eval");
static_assert(offsetof(FastSmem, eid) == offsetof(FastSmem, eval) + sizeof(float) * kExcCap &&
                  offsetof(FastSmem, lkey) == 4 * kPresRegion,
              "ccnt .. eid must be contiguous");
static_assert(kExcCap <= 2 * kThreads, "two ranks per thread");

// Block b of a 16-byte-aligned row whose block is wholly inside it, as loaded (one
// unconditional vector load, so that several in flight are waited for together: Row::load's
// per-lane range test puts each load behind a branch), and its values.
template <class Tin>
struct WholeBlock;
template <>
struct WholeBlock<uint16_t> {
  uint4 d;
  __device__ __forceinline__ void load(const uint16_t* p, int b) { d = *reinterpret_cast<const uint4*>(p + b * kBlk); }
  __device__ __forceinline__ void values(float v[kBlk]) const {
    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};
template <>
struct WholeBlock<float> {
  float4 d0, d1;
  __device__ __forceinline__ void load(const float* p, int b) {
    d0 = *reinterpret_cast<const float4*>(p + b * kBlk);
    d1 = *reinterpret_cast<const float4*>(p + b * kBlk + 4);
  }
  __device__ __forceinline__ void values(float v[kBlk]) const {
    v[0] = d0.x; v[1] = d0.y; v[2] = d0.z; v[3] = d0.w;
    v[4] = d1.x; v[5] = d1.y; v[6] = d1.z; v[7] = d1.w;
  }
};

template <class Tin>
struct Row {
  const Tin* p;
  int V;
  int nblk;
  int nstripes;
  bool vec;
  const uint8_t* bm;   // per-block lane masks of exceptions, or null
  const int32_t* eid;  // exceptions of this row (in no particular order)
  const float* eval;
  int nexc;

  // Values of block b and the lanes that hold bulk (non-exception, in-range) values.
  __device__ __forceinline__ uint32_t load(int b, float v[kBlk]) const;
};

template <>
__device__ __forceinline__ uint32_t Row<uint16_t>::load(int b, float v[kBlk]) const {
  const int base = b * kBlk;
  uint32_t valid;
  if (vec && base + kBlk <= V) {
    const uint4 d = *reinterpret_cast<const uint4*>(p + base);
    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
    valid = 0xFFu;
  } else {
    valid = 0;
#pragma unroll
    for (int i = 0; i < kBlk; ++i) {
      const bool in = base + i < V;
      v[i] = in ? bf16_to_f32(p[base + i]) : 0.0f;
      valid |= (in ? 1u : 0u) << i;
    }
  }
  if (bm) valid &= ~static_cast<uint32_t>(bm[b]);
  return valid;
}

template <>
__device__ __forceinline__ uint32_t Row<float>::load(int b, float v[kBlk]) const {
  const int base = b * kBlk;
  uint32_t valid;
  if (vec && base + kBlk <= V) {
    const float4 d0 = *reinterpret_cast<const float4*>(p + base);
    const float4 d1 = *reinterpret_cast<const float4*>(p + base + 4);
    v[0] = d0.x; v[1] = d0.y; v[2] = d0.z; v[3] = d0.w;
    v[4] = d1.x; v[5] = d1.y; v[6] = d1.z; v[7] = d1.w;
    valid = 0xFFu;
  } else {
    valid = 0;
#pragma unroll
    for (int i = 0; i < kBlk; ++i) {
      const bool in = base + i < V;
      v[i] = in ? p[base + i] : 0.0f;
      valid |= (in ? 1u : 0u) << i;
    }
  }
  if (bm) valid &= ~static_cast<uint32_t>(bm[b]);
  return valid;
}

// Stripes in flight in for_each_block_ahead's rolling window (0: groups of kDepth stripes, each
// group's loads issued together and used before the next group's).
constexpr int kRollDepth = 2;

// The IEEE maximum of a block's eight values (NaN when one of them is; -0 below +0), as a chain
// that compiles to four three-operand maxima (v_maximum3_f32).
__device__ __forceinline__ float max_of8(const float (&x)[kBlk]) {
  float r = x[0];
#pragma unroll
  for (int i = 1; i < kBlk; ++i) r = __builtin_elementwise_maximum(r, x[i]);
  return r;
}

// Every block of the row once, as fb(v, out, b) in the calling thread: v its eight values and
// `out` the lanes that hold no bulk value (penalised, or past the row's end). The groups of kDepth
// stripes wholly inside an aligned row have their loads (and lane masks) issued together, ahead
// of the work on them. Exceptions are the caller's.
template <class Tin, class FB>
__device__ __forceinline__ void for_each_block_ahead(const Row<Tin>& row, FB fb, int j0 = 0) {
  constexpr int kDepth = 2;  // (measured on logprobs and fp32 rows: 2 beats 4 and 8)
  const int whole = row.vec ? row.V / kBlk / kThreads : 0;  // (uniform) such stripes
  int j = j0;  // (the stripes below j0, a multiple of kDepth, were visited by the caller)
  if constexpr (kRollDepth > 0) {
    // a rolling window: as stripe j's values are taken out of slot k, the slot's next load
    // (stripe j + kRollDepth) is issued, so kRollDepth stripes stay in flight
    constexpr int D = kRollDepth;
    const int end = j0 + (whole - j0) / D * D;  // (uniform)
    if (end > j0) {
      WholeBlock<Tin> q[D];
      uint32_t masked[D];
#pragma clang loop unroll(full)
      for (int k = 0; k < D; ++k) {
        const int b = (j0 + k) * kThreads + threadIdx.x;
        q[k].load(row.p, b);
        masked[k] = row.bm ? row.bm[b] : 0u;
      }
      for (; j < end; j += D) {
#pragma clang loop unroll(full)
        for (int k = 0; k < D; ++k) {
          const int b = (j + k) * kThreads + threadIdx.x;
          float v[kBlk];
          q[k].values(v);
          const uint32_t m = masked[k];
          // (the last window reloads its own stripes: in bounds, and never used)
          const int bn = (j + D + k < end ? j + D + k : j + k) * kThreads + threadIdx.x;
          q[k].load(row.p, bn);
          masked[k] = row.bm ? row.bm[bn] : 0u;
          fb(v, m, b);
        }
      }
    }
  }
  for (; j + kDepth <= whole; j += kDepth) {
    WholeBlock<Tin> q[kDepth];
    uint32_t masked[kDepth];
#pragma clang loop unroll(full)
    for (int k = 0; k < kDepth; ++k) {
      const int b = (j + k) * kThreads + threadIdx.x;
      q[k].load(row.p, b);
      masked[k] = row.bm ? row.bm[b] : 0u;
    }
#pragma clang loop unroll(full)
    for (int k = 0; k < kDepth; ++k) {
      const int b = (j + k) * kThreads + threadIdx.x;
      float v[kBlk];
      q[k].values(v);
      fb(v, masked[k], b);
    }
  }
  for (int b = j * kThreads + threadIdx.x; b < row.nblk; b += kThreads) {
    float v[kBlk];
    const uint32_t valid = row.load(b, v);
    fb(v, ~valid & 0xFFu, b);
  }
}

// Visit every element of the row once: bulk lanes through `f(x, id)` in the calling thread's
// blocks, exceptions spread over the workgroup.
template <class Tin, class F>
__device__ __forceinline__ void for_each_ahead(const Row<Tin>& row, F f, int j0 = 0) {
  for_each_block_ahead(row, [&](const float (&v)[kBlk], uint32_t out, int b) {
#pragma unroll
    for (int i = 0; i < kBlk; ++i)
      if (!(out & (1u << i))) f(v[i], b * kBlk + i);
  }, j0);
  for (int e = threadIdx.x; e < row.nexc; e += kThreads) f(row.eval[e], row.eid[e]);
}

// The same visit, one block at a time.
template <class Tin, class F>
__device__ __forceinline__ void for_each_plain(const Row<Tin>& row, F f) {
  for (int b = threadIdx.x; b < row.nblk; b += kThreads) {
    float v[kBlk];
    const uint32_t valid = row.load(b, v);
#pragma unroll
    for (int i = 0; i < kBlk; ++i)
      if (valid & (1u << i)) f(v[i], b * kBlk + i);
  }
  for (int e = threadIdx.x; e < row.nexc; e += kThreads) f(row.eval[e], row.eid[e]);
}

// The sampling kernels' visit: loads ahead for fp32 rows; bf16 rows, which reach it only off the
// fast path, one block at a time (the loads-ahead code there measured 0.5 us slower on the fast
// path's own launches, through the kernel's code size).
template <class Tin, class F>
__device__ __forceinline__ void for_each(const Row<Tin>& row, F f) {
  if constexpr (sizeof(Tin) == 4)
    for_each_ahead(row, f);
  else
    for_each_plain(row, f);
}

// The penalised logit of token d (bulk or exception); all threads call, all get the value.
template <class Tin>
__device__ __forceinline__ float value_of(const Row<Tin>& row, int d, float* slot) {
  if (threadIdx.x == 0) *slot = load_one<Tin>(row.p, d);
  lds_barrier();
  for (int e = threadIdx.x; e < row.nexc; e += kThreads)
    if (row.eid[e] == d) *slot = row.eval[e];
  lds_barrier();
  const float v = *slot;
  lds_barrier();
  return v;
}

// Fill `words` (V / 8 bytes, one lane mask per 8-id block) with the row's penalised ids.
template <class Tin>
__device__ __forceinline__ void build_bitmap(Row<Tin>& row, uint32_t* words) {
  const int nw = (row.nblk + 3) / 4;
  for (int i = threadIdx.x; i < nw; i += kThreads) words[i] = 0;
  lds_barrier();
  // (row.eid: the workspace on the generic path, LDS on the fast path)
  for_each_id<false>(row.eid, row.nexc, [&](int v, int) {
    const uint32_t id = static_cast<uint32_t>(v);
    atomicOr(&words[id >> 5], 1u << (id & 31u));
  });
  lds_barrier();
  row.bm = reinterpret_cast<const uint8_t*>(words);
}

// Add 1 to hist[digit] for every lane with `valid`, pre-aggregating up to four repeated digits
// per wave with ballots (the top digits of N(0, s) logits fall into a handful of bins).
__device__ __forceinline__ void hist_count(uint32_t* hist, uint32_t digit, bool valid) {
  u64 active = __ballot(valid);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    if (!active) break;
    const int leader = __ffsll(static_cast<long long>(active)) - 1;
    const uint32_t d0 = __builtin_amdgcn_readlane(digit, leader);
    const u64 same = __ballot(valid && digit == d0);
    if (lane_id() == leader) atomicAdd(&hist[d0], static_cast<uint32_t>(__popcll(same)));
    if (digit == d0) valid = false;
    active &= ~same;
  }
  if (valid) atomicAdd(&hist[digit], 1u);
}

__device__ __forceinline__ void hist_mass(uint32_t* hc, u64* hm, uint32_t digit, u64 q, bool valid) {
  u64 active = __ballot(valid);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    if (!active) break;
    const int leader = __ffsll(static_cast<long long>(active)) - 1;
    const uint32_t d0 = __builtin_amdgcn_readlane(digit, leader);
    const bool mine = valid && digit == d0;
    const u64 same = __ballot(mine);
    const u64 s = wave_sum<u64>(mine ? q : 0ull);
    if (lane_id() == leader) {
      atomicAdd(&hc[d0], static_cast<uint32_t>(__popcll(same)));
      atomicAdd(&hm[d0], s);
    }
    if (mine) valid = false;
    active &= ~same;
  }
  if (valid) {
    atomicAdd(&hc[digit], 1u);
    atomicAdd(&hm[digit], q);
  }
}

// Smallest key K in [lo, hi] with pred(val_of(K)); pred(val_of(hi)) must hold and pred must be
// monotone over the keys of [lo, hi]. One wave searches (every lane calls, every lane gets the
// key): each round tests 64 keys spread over [lo, hi] and keeps the span between the last
// failing and the first passing one, so a 32-bit range takes 6 rounds where a bisection takes 32
// serial steps.
template <class P>
__device__ __forceinline__ uint32_t bisect_key_wave(uint32_t lo, uint32_t hi, P pred) {
  const u64 l1 = static_cast<u64>(lane_id()) + 1u;
  while (lo < hi) {  // (uniform)
    const u64 span = hi - lo;
    const uint32_t probe = lo + static_cast<uint32_t>((span * l1) >> 6);  // lane 63 probes hi
    const u64 ok = __ballot(pred(val_of(probe)));
    const int f = __ffsll(static_cast<long long>(ok)) - 1;  // (lane 63's probe always passes)
    const uint32_t hi2 = __builtin_amdgcn_readlane(probe, f);
    const uint32_t below = __builtin_amdgcn_readlane(probe, f > 0 ? f - 1 : 0);
    lo = f > 0 ? below + 1u : lo;
    hi = hi2;
  }
  return hi;
}

// First element index (ascending id) where the running count of w(x, id) (0 or 1) exceeds
// `target` (clamped to total - 1). Returns -1 when no element has w = 1.
template <class Tin, class W>
__device__ __forceinline__ int find_first(const Row<Tin>& row, W wf, u64 target, Search& s) {
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  // 1. per-(wave, stripe) counts, four stripes' loads in flight per thread
  for (int j0 = 0; j0 < row.nstripes; j0 += 4) {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int b = (j0 + k) * kThreads + tid;
      if (j0 + k < row.nstripes && b < row.nblk) {
        float v[kBlk];
        const uint32_t valid = row.load(b, v);
#pragma unroll
        for (int i = 0; i < kBlk; ++i)
          if (valid & (1u << i)) w[k] += static_cast<uint32_t>(wf(v[i], b * kBlk + i));
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t ws = wave_sum<uint32_t>(w[k]);
      if (lane_id() == 0 && j0 + k < row.nstripes) s.cell[wv][j0 + k] = ws;
    }
  }
  __syncthreads();
  for (int e = tid; e < row.nexc; e += kThreads) {
    const int id = row.eid[e];
    const u64 w = wf(row.eval[e], id);
    if (w) {
      const int b = id / kBlk;
      atomicAdd(&s.cell[(b % kThreads) / kWave][b / kThreads], w);
    }
  }
  __syncthreads();
  // 2. stripe totals, prefix over stripes, the stripe where the count crosses the target
  if (wv == 0) {
    const int j = lane_id();
    u64 t = 0;
    if (j < row.nstripes)
      for (int w = 0; w < kWaves; ++w) t += s.cell[w][j];
    const u64 inc = wave_incl_scan<u64>(t);
    const u64 total = dpp::last(inc);
    u64 tg = target;
    if (total > 0 && tg > total - 1) tg = total - 1;
    const bool hit = total > 0 && inc > tg && (inc - t) <= tg;
    const u64 hm = __ballot(hit);
    if (j == 0) {
      s.bq[0] = total;
      s.bq[1] = tg;
      s.bi[0] = hm ? (__ffsll(static_cast<long long>(hm)) - 1) : -1;
    }
    if (hit) s.bq[2] = inc - t;  // count before stripe js
  }
  __syncthreads();
  const u64 total = s.bq[0];
  if (total == 0) {
    __syncthreads();
    return -1;
  }
  const u64 tg = s.bq[1];
  const int js = s.bi[0] < 0 ? 0 : s.bi[0];
  const u64 base = s.bi[0] < 0 ? 0ull : s.bq[2];
  // 3. per-thread counts inside stripe js, prefix over threads
  {
    const int b = js * kThreads + tid;
    u64 w = 0;
    if (b < row.nblk) {
      float v[kBlk];
      const uint32_t valid = row.load(b, v);
#pragma unroll
      for (int i = 0; i < kBlk; ++i)
        if (valid & (1u << i)) w += wf(v[i], b * kBlk + i);
    }
    s.tw[tid] = w;
  }
  if (tid < kBlk) s.slot[tid] = 0;
  if (tid == 0) {
    s.slot_mask = 0;
    s.bi[1] = 0;  // overwritten by the thread whose range holds the target
    s.bq[3] = base;
  }
  __syncthreads();
  for (int e = tid; e < row.nexc; e += kThreads) {
    const int id = row.eid[e];
    const int b = id / kBlk;
    if (b / kThreads == js) {
      const u64 w = wf(row.eval[e], id);
      if (w) atomicAdd(&s.tw[b % kThreads], w);
    }
  }
  __syncthreads();
  {
    const u64 w = s.tw[tid];
    u64 tot2;
    const u64 ex = block_excl_scan<u64>(w, s.red64, &tot2);
    if (w > 0 && base + ex <= tg && base + ex + w > tg) {
      s.bi[1] = tid;
      s.bq[3] = base + ex;
    }
  }
  __syncthreads();
  const int ts = s.bi[1];
  const int bs = js * kThreads + ts;
  const u64 base2 = s.bq[3];
  // 4. the exceptions of block bs, then one thread walks its eight lanes
  for (int e = tid; e < row.nexc; e += kThreads) {
    const int id = row.eid[e];
    if (id / kBlk == bs) {
      s.slot[id % kBlk] = wf(row.eval[e], id);
      atomicOr(&s.slot_mask, 1u << (id % kBlk));
    }
  }
  __syncthreads();
  if (tid == 0) {
    float v[kBlk];
    const uint32_t valid = row.load(bs, v);
    u64 c = base2;
    int found = bs * kBlk;
    for (int i = 0; i < kBlk; ++i) {
      u64 w = 0;
      if (s.slot_mask & (1u << i)) w = s.slot[i];
      else if (valid & (1u << i)) w = wf(v[i], bs * kBlk + i);
      c += w;
      if (c > tg) {
        found = bs * kBlk + i;
        break;
      }
    }
    s.bi[2] = found;
  }
  __syncthreads();
  const int res = s.bi[2];
  __syncthreads();
  return res;
}

// ---- generic path: radix descents over 32-bit ordered keys ------------------------------------

// The key of the kth largest element (k >= 1).
template <class Tin>
__device__ uint32_t radix_kth(const Row<Tin>& row, const CandList* list, uint32_t k, Radix& s) {
  uint32_t prefix = 0;
  uint32_t kk = k;
  for (int lvl = 0; lvl < 4; ++lvl) {
    const int shift = 24 - 8 * lvl;
    for (int i = threadIdx.x; i < 256; i += kThreads) s.hcnt[i] = 0;
    if (threadIdx.x == 0) {
      s.bk[0] = 0;
      s.bk[1] = 0;
    }
    __syncthreads();
    const bool all = lvl == 0;
    const uint32_t pfx = prefix;
    // (every lane calls hist_count each round: its ballots need the whole wave)
    if (list) {
      for (int i0 = 0; i0 < list->n; i0 += kThreads) {
        const int i = i0 + threadIdx.x;
        const bool ok = i < list->n;
        const uint32_t key = key_of(ok ? list->c[i].x : 0.0f);
        hist_count(s.hcnt, (key >> shift) & 255u, ok && (all || (key >> (shift + 8)) == pfx));
      }
    } else {
      for (int b = threadIdx.x, j = 0; j < row.nstripes; ++j, b += kThreads) {
        float v[kBlk];
        const uint32_t valid = b < row.nblk ? row.load(b, v) : 0u;
#pragma unroll
        for (int i = 0; i < kBlk; ++i) {
          const uint32_t key = key_of(v[i]);
          const bool m = (valid & (1u << i)) && (all || (key >> (shift + 8)) == pfx);
          hist_count(s.hcnt, (key >> shift) & 255u, m);
        }
      }
      for (int e0 = 0; e0 < row.nexc; e0 += kThreads) {
        const int e = e0 + threadIdx.x;
        const bool ok = e < row.nexc;
        const uint32_t key = key_of(ok ? row.eval[e] : 0.0f);
        const bool m = ok && (all || (key >> (shift + 8)) == pfx);
        hist_count(s.hcnt, (key >> shift) & 255u, m);
      }
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
      // lane l covers digits 255-4l .. 252-4l (descending)
      const int l = lane_id();
      uint32_t c[4], cs = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = s.hcnt[255 - 4 * l - i];
        cs += c[i];
      }
      const uint32_t inc = wave_incl_scan<uint32_t>(cs);
      uint32_t above = inc - cs;
      if (above < kk && inc >= kk) {
        for (int i = 0; i < 4; ++i) {
          if (above + c[i] >= kk) {
            s.bk[0] = 255 - 4 * l - i;
            s.bk[1] = above;
            break;
          }
          above += c[i];
        }
      }
    }
    __syncthreads();
    prefix = (prefix << 8) | s.bk[0];
    kk -= s.bk[1];
    __syncthreads();
  }
  return prefix;
}

enum MassMode { kCutoff = 0, kCross = 1 };

// Radix descent on masses among elements with x >= x0.
//   kCutoff: the lowest value whose mass strictly above is < target (the top-p cutoff)
//   kCross : the value whose group holds the target: above <= target < above + group mass
// Returns the value's key; *n_c its count, *mass_c its group mass, *m_above the mass above it.
template <class Tin>
__device__ uint32_t radix_mass(const Row<Tin>& row, const CandList* list, int mode, float x0, float T, float mz,
                               double target, Radix& s, uint32_t* n_c, u64* mass_c, u64* m_above,
                               uint32_t prefix0 = 0, int bits0 = 0, u64 mprev0 = 0) {
  // the descent starts below a known prefix of bits0 key bits (the elements above it hold mass
  // mprev0), then takes digits of up to 8 bits
  uint32_t prefix = prefix0;
  u64 mprev = mprev0;
  for (int done = bits0; done < 32;) {
    const int width = 32 - done < 8 ? 32 - done : 8;
    const int shift = 32 - done - width;
    const uint32_t dmask = (1u << width) - 1u;
    const bool all = done == 0;
    for (int i = threadIdx.x; i < 256; i += kThreads) {
      s.hcnt[i] = 0;
      s.hmass[i] = 0;
    }
    if (threadIdx.x == 0) {
      s.bk[0] = 0;
      s.bk[1] = 0;
      s.bq[0] = mprev;
      s.bq[1] = 0;
    }
    __syncthreads();
    auto one = [&](float x, bool valid) {
      const uint32_t key = key_of(x);
      const bool m = valid && x >= x0 && (all || (key >> (shift + width)) == prefix);
      const u64 q = m ? mass_q(ptilde(x, T, mz)) : 0ull;
      hist_mass(s.hcnt, s.hmass, (key >> shift) & dmask, q, m);
    };
    // (every lane calls `one` each round: its ballots and wave sums need the whole wave)
    if (list) {
      for (int i0 = 0; i0 < list->n; i0 += kThreads) {
        const int i = i0 + threadIdx.x;
        const bool ok = i < list->n;
        one(ok ? list->c[i].x : 0.0f, ok);
      }
    } else {
      for (int b = threadIdx.x, j = 0; j < row.nstripes; ++j, b += kThreads) {
        float v[kBlk];
        const uint32_t valid = b < row.nblk ? row.load(b, v) : 0u;
#pragma unroll
        for (int i = 0; i < kBlk; ++i) one(v[i], valid & (1u << i));
      }
      for (int e0 = 0; e0 < row.nexc; e0 += kThreads) {
        const int e = e0 + threadIdx.x;
        const bool ok = e < row.nexc;
        one(ok ? row.eval[e] : 0.0f, ok);
      }
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
      const int l = lane_id();
      u64 ms = 0;
      uint32_t c[4];
      u64 mm[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = s.hcnt[255 - 4 * l - i];
        mm[i] = s.hmass[255 - 4 * l - i];
        ms += mm[i];
      }
      const u64 inc = wave_incl_scan<u64>(ms);
      u64 above = mprev + inc - ms;
      int cand = -1;
      u64 cand_above = 0;
      uint32_t cand_c = 0;
      u64 cand_m = 0;
      for (int i = 0; i < 4; ++i) {
        const double ab = static_cast<double>(above);
        const bool ok = mode == kCutoff ? (ab < target && c[i] > 0)
                                        : (c[i] > 0 && ab <= target && target < static_cast<double>(above + mm[i]));
        if (ok) {
          cand = 255 - 4 * l - i;
          cand_above = above;
          cand_c = c[i];
          cand_m = mm[i];
        }
        above += mm[i];
      }
      // kCutoff: the lowest candidate digit = the highest lane with one; kCross: the unique one
      const u64 hm = __ballot(cand >= 0);
      const int lw = hm ? 63 - __clzll(static_cast<long long>(hm)) : -1;
      if (l == lw) {
        s.bk[0] = static_cast<uint32_t>(cand);
        s.bq[0] = cand_above;
        s.bk[1] = cand_c;
        s.bq[1] = cand_m;
      }
    }
    __syncthreads();
    prefix = (prefix << width) | s.bk[0];
    mprev = s.bq[0];
    *n_c = s.bk[1];
    *mass_c = s.bq[1];
    __syncthreads();
    done += width;
  }
  *m_above = mprev;
  return prefix;
}

// What a row's filters left: kept(x, id) = x >= x0 && (!partial || x > vc || (x == vc && id <=
// idr)); S the kept mass; a point mass at `point` for greedy and degenerate rows.
struct Kept {
  float x0 = -INFINITY;
  float vc = 0.0f;
  bool partial = false;
  int idr = 0;
  uint32_t r = 0;    // kept members of the cutoff group
  u64 mabove_c = 0;  // mass strictly above the cutoff value
  u64 qc = 0;        // mass of one member of the cutoff group
  bool has_cut = false;
  u64 S = 0;
  int point = -1;

  __device__ __forceinline__ bool keep(float x, int id) const {
    if (!(x >= x0)) return false;
    if (!partial) return true;
    return x > vc || (x == vc && id <= idr);
  }
};


// Greedy rows and rows whose scaled logits are not all finite: a point mass. Shared by both
// paths; returns true when the row is such a row (and sets k.point).
template <class Tin>
__device__ __forceinline__ bool degenerate(const Row<Tin>& row, const RowParams& p, uint32_t mkey, int imax, float mz,
                           Search& s, Kept& k) {
  if (!(p.T > 0.0f) || mkey == 0xFFFFFFFFu) {
    k.point = imax;  // greedy (sampler.py:70-71), or a NaN logit: its first index
    return true;
  }
  const float T = p.T;
  if (mz != mz) {  // x = +inf with T = +inf: the first index where z is NaN
    k.point = find_first(row, [&](float x, int) -> u64 { const float z = x / T; return z != z; }, 0ull, s);
    return true;
  }
  if (mz == INFINITY) {
    k.point = find_first(row, [&](float x, int) -> u64 { return x / T == INFINITY; }, 0ull, s);
    return true;
  }
  if (mz == -INFINITY) {
    k.point = 0;
    return true;
  }
  return false;
}

// Writes the row's outputs: probabilities (probs mode) or the sampled id and draft probability,
// and with STATE the row's RowState. `draw` is the drawn token (ignored for point rows).
template <bool STATE, class Tin>
__device__ __forceinline__ void finish(const SampleArgs& a, const Row<Tin>& row, const RowParams& p, float mz,
                       const Kept& k, int draw, float* vslot, int r) {
  const int tid = threadIdx.x;
  if (STATE && tid == 0) {
    RowState st;
    st.mz = mz;
    st.T = p.T;
    st.x0 = k.x0;
    st.vc = k.vc;
    st.partial = k.partial;
    st.idr = k.idr;
    st.point = k.point;
    st.pad = 0;
    st.S = k.S;
    a.out_state[r] = st;
  }
  if (a.out_probs) {
    float* o = a.out_probs + static_cast<int64_t>(r) * a.probs_stride;
    if (k.point >= 0) {
      for (int i = tid; i < row.V; i += kThreads) o[i] = i == k.point ? 1.0f : 0.0f;
      return;
    }
    const double inv = kMassScale / static_cast<double>(k.S);
    const float T = p.T;
    for_each(row, [&](float x, int id) {
      o[id] = k.keep(x, id) ? static_cast<float>(ptilde(x, T, mz) * inv) : 0.0f;
    });
    return;
  }
  int tok;
  double dprob = 0.0;
  if (k.point >= 0) {
    tok = k.point;
    dprob = p.draft == tok ? 1.0 : 0.0;
  } else {
    tok = draw;
    if (p.draft >= 0 && p.draft < row.V && a.out_dprob) {
      const float xd = value_of(row, p.draft, vslot);
      if (k.keep(xd, p.draft)) dprob = ptilde(xd, p.T, mz) * kMassScale / static_cast<double>(k.S);
    }
  }
  if (tid == 0) {
    a.out_ids[r] = tok;
    if (a.out_dprob) a.out_dprob[r] = static_cast<float>(dprob);
    if (a.hist_out) a.hist_out[p.h1] = tok;  // (STATE launches carry no history: never set there)
  }
}

// With the cutoff group partial, the id of its r-th member (what kept() needs): only probs mode
// and a draft token inside that group ask for it.
template <bool STATE, class Tin>
__device__ __forceinline__ void resolve_idr(const SampleArgs& a, const Row<Tin>& row, const RowParams& p, Kept& k,
                            Search& s) {
  if (!k.partial) return;
  bool need = STATE || a.out_probs != nullptr;
  if (!need && p.draft >= 0 && p.draft < row.V && a.out_dprob) need = value_of(row, p.draft, &s.vslot) == k.vc;
  if (need) {
    const float vc = k.vc;
    k.idr = find_first(row, [&](float x, int) -> u64 { return x == vc; }, static_cast<u64>(k.r - 1), s);
  }
}

// ---- generic path -----------------------------------------------------------------------------
// The generic path's chunk masses: chunk c holds the keys whose top 10 bits are 1023 - c (so
// chunk 0 holds the largest values). Wave 0 picks the chunk a mass descent starts in and the
// mass above it, with the comparisons radix_mass makes on its digits:
//   kCutoff: the last chunk holding mass whose mass above is < target;
//   kCross : the chunk with mass above <= target < mass above + its mass.
// Lane l sums chunks 16l .. 16l + 15; the chunks of one lane are then searched across a 16-lane
// row. Returns -1 when no chunk qualifies (the caller descends over the whole row instead).
__device__ __forceinline__ int chunk_pick(const u64* cm, int mode, double target, u64* above_out) {
  const int l = lane_id();
  u64 sum = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) sum += cm[16 * l + q];
  const u64 incl = wave_incl_scan<u64>(sum);
  const u64 base = incl - sum;
  int L = -1;
  if (mode == kCutoff) {
    // the chunks with mass above < target are a prefix: the last lane starting below it when
    // that lane holds mass, else the last lane before it holding mass
    const u64 below = __ballot(static_cast<double>(base) < target);
    if (below) {
      const int lb = 63 - __clzll(static_cast<long long>(below));
      const u64 held = __ballot(sum > 0 && l <= lb);
      L = held ? 63 - __clzll(static_cast<long long>(held)) : -1;
    }
  } else {
    const u64 hl = __ballot(sum > 0 && static_cast<double>(base) <= target && target < static_cast<double>(base + sum));
    L = hl ? __ffsll(static_cast<long long>(hl)) - 1 : -1;
  }
  if (L < 0) return -1;
  const u64 mq = cm[16 * L + (l & 15)];
  const u64 run = readlane64(base, L) + row_incl_scan<u64>(mq) - mq;
  u64 hm;
  if (mode == kCutoff) {
    hm = __ballot(mq > 0 && static_cast<double>(run) < target) & 0xFFFFull;
    if (!hm) return -1;
    const int q = 63 - __clzll(static_cast<long long>(hm));
    *above_out = readlane64(run, q);
    return 16 * L + q;
  }
  hm = __ballot(mq > 0 && static_cast<double>(run) <= target && target < static_cast<double>(run + mq)) & 0xFFFFull;
  if (!hm) return -1;
  const int q = __ffsll(static_cast<long long>(hm)) - 1;
  *above_out = readlane64(run, q);
  return 16 * L + q;
}

// ---- generic path: small top-k lists, sorted ---------------------------------------------------
// A top-k candidate list of at most kSortCap elements is sorted once, by descending value and
// then ascending id (the draw's order), and the rest of the row's work reads it by index: the
// K-th largest is entry K - 1, and wave 0 alone finds the top-p cutoff group and the drawn
// element from the exclusive prefix of the masses, with the comparisons the radix descents make
// on their digits (so both give the same groups; see sorted_tail).
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

constexpr int kSortCap = 256;  // four entries per lane of wave 0
// Streaming top-k candidates (fp32 rows): K at most kStreamK, at most kStreamCap staged elements
// (in LDS after the candidate list: the sort's staging, unused until then).
constexpr int kStreamK = 384;
constexpr int kStreamCap = 1536;
static_assert(kMatchOffset + 2 * kCandCap + 2 * kStreamCap <= kChunk, "the staged candidates must fit");
static_assert(kMatchOffset + 2 * kCandCap + 2 * kSortCap <= kChunk, "the sort's staging must fit");

// Sorts c[0, n), n <= kSortCap, in place (rank by counting; tmp holds n entries). Every thread
// calls; the sorted list is visible on return. The order is one 64-bit key per entry, ordered key
// above the complemented id (larger first: larger value, then smaller id), staged in tmp; each
// entry's rank is the count of larger keys, and it is written there (every read of c is done
// before the first barrier).
__device__ __forceinline__ void sort_cands(Cand* c, int n, Cand* tmp) {
  const int i = threadIdx.x;
  u64* kk = reinterpret_cast<u64*>(tmp);
  static_assert(sizeof(Cand) == sizeof(u64), "one staged key per entry");
  Cand me{0.0f, 0};
  u64 km = 0;
  if (i < n) {
    me = c[i];
    km = (static_cast<u64>(key_of(me.x)) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(me.id));
    kk[i] = km;
  }
  lds_barrier();
  if (i < n) {
    uint32_t rank = 0;
    for (int j = 0; j < n; ++j) rank += kk[j] > km ? 1u : 0u;  // (j uniform: one broadcast read per wave)
    c[rank] = me;
  }
  lds_barrier();
}

// floor(a / b) for a < 2^53 and b > 0 (both exact in fp64): the fp64 quotient is at most one
// above it (a representable integer quotient is exact, and rounding is monotonic), corrected by
// one integer product.
__device__ __forceinline__ u64 udiv53(u64 a, u64 b) {
  u64 q = static_cast<u64>(static_cast<double>(a) / static_cast<double>(b));
  if (q * b > a) --q;
  return q;
}

// Top-p cutoff and draw over a sorted list c[0, n) that holds every element >= k.x0 (the kept
// set is a prefix of it). Wave 0 computes; on success the results reach k and the row's outputs
// are written (returns true); when no group qualifies as the cutoff (which the radix descent
// would resolve on its own terms) nothing is changed and it returns false.
//
// Equivalence with radix_mass: with E_i the exclusive prefix of the masses in list order, a
// digit's or a key group's "mass above" is E at its first element. kCutoff keeps the lowest group
// whose double(E) < P: the E are non-decreasing, so that is the group of the last element with
// double(E_i) < P. kCross takes the group with double(E_g) <= t < double(E_g + M_g); those
// intervals tile [0, double(S)), and so do the elements' [double(E_i), double(E_i + q_i)) inside
// them, so it is the group of the one element whose interval holds t.
template <bool STATE, class Tin>
__device__ __forceinline__ bool sorted_tail(const SampleArgs& a, const Row<Tin>& row, const RowParams& p,
                                            GenericSmem& g, Search& s, const Cand* c, int n, float mz, Kept& k,
                                            int r) {
  // results: hcnt[0] ok, [1] cutoff key, [2] first index of the cutoff group, [3] its size,
  // [4] kept members r, [5] partial, [6] draw index; bq[0] S, bq[1] mass above the cutoff,
  // bq[2] mass of one member of the cutoff group
  uint32_t* res = g.rdx.hcnt;
  u64* resq = g.rdx.bq;
  // every entry's mass, one per thread (rdx.hmass holds kSortCap), for wave 0
  const uint32_t k0 = key_of(k.x0);
  {
    const int i = threadIdx.x;
    if (i < n) {
      const float x = c[i].x;
      g.rdx.hmass[i] = key_of(x) >= k0 ? mass_q(ptilde(x, p.T, mz)) : 0ull;
    }
  }
  static_assert(sizeof(g.rdx.hmass) / sizeof(u64) >= kSortCap, "a mass per sorted entry");
  lds_barrier();
  if (threadIdx.x < kWave) {
    const int l = lane_id();
    uint32_t key[4];
    u64 q[4];
    u64 ls = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int i = 4 * l + t;
      const float x = i < n ? c[i].x : 0.0f;
      const bool in = i < n && key_of(x) >= k0;
      key[t] = in ? key_of(x) : 0u;  // (0: below every kept key)
      q[t] = in ? g.rdx.hmass[i] : 0ull;
      ls += q[t];
    }
    const u64 incl = wave_incl_scan<u64>(ls);
    u64 E[4];
    E[0] = incl - ls;
#pragma unroll
    for (int t = 1; t < 4; ++t) E[t] = E[t - 1] + q[t - 1];
    const u64 S0 = dpp::last(incl);
    // entry i's value of a per-slot array (i uniform): slot i mod 4 of lane i / 4
    auto at64 = [&](const u64 (&v)[4], uint32_t i) {
      const uint32_t t = i & 3u;
      return readlane64(t == 0u ? v[0] : t == 1u ? v[1] : t == 2u ? v[2] : v[3], static_cast<int>(i >> 2));
    };
    // one key group of the kept prefix (a kept key, gk != 0): its first index (the kept elements
    // with a larger key, all before it), its size and the mass above it (E at its first index);
    // its members are contiguous and have one mass, returned in q1
    auto group = [&](uint32_t gk, uint32_t* f, uint32_t* cnt, u64* above, u64* q1) {
      uint32_t first = 0xFFFFFFFFu, m = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const u64 b = __ballot(key[t] == gk);
        m += static_cast<uint32_t>(__popcll(b));
        const uint32_t i = b ? 4u * static_cast<uint32_t>(__ffsll(static_cast<long long>(b)) - 1) + t : 0xFFFFFFFFu;
        first = i < first ? i : first;
      }
      *f = first;
      *cnt = m;
      *above = at64(E, first);
      *q1 = at64(q, first);
    };
    bool ok = true;
    u64 S = S0;
    uint32_t ck = 0, fc = 0, nc = 0, rr = 0;
    u64 mabove = 0, qc = 0;
    bool partial = false, has_cut = false;
    if (p.tp < 1.0f) {
      const double P = static_cast<double>(p.tp) * static_cast<double>(S0);
      uint32_t below = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) below += key[t] != 0u && static_cast<double>(E[t]) < P ? 1u : 0u;
      const uint32_t nb = wave_sum<uint32_t>(below);
      ok = nb > 0;
      if (ok) {
        const uint32_t js = nb - 1u;  // the last element with E < P
        const uint32_t tj = js & 3u;
        ck = __builtin_amdgcn_readlane(tj == 0u ? key[0] : tj == 1u ? key[1] : tj == 2u ? key[2] : key[3],
                                       static_cast<int>(js >> 2));
        group(ck, &fc, &nc, &mabove, &qc);
        rr = nc;
        if (qc > 0) {
          const double cr = ceil((P - static_cast<double>(mabove)) / static_cast<double>(qc));
          rr = cr < 1.0 ? 1u : (cr >= static_cast<double>(nc) ? nc : static_cast<uint32_t>(cr));
        }
        partial = rr < nc;
        has_cut = true;
        S = mabove + static_cast<u64>(rr) * qc;
      }
    }
    uint32_t di = 0;
    if (ok && !a.out_probs) {
      const u64 td = static_cast<u64>(static_cast<double>(p.u) * static_cast<double>(S));
      const u64 tdc = td < S ? td : S - 1;
      if (has_cut && tdc >= mabove && qc > 0) {
        di = fc + static_cast<uint32_t>(udiv53(tdc - mabove, qc));
      } else {
        // the group holding tdc among the elements >= x0 (x0 raised to the cutoff value when
        // the cutoff group is whole)
        const uint32_t kx = has_cut && !partial ? ck : k0;
        const double tt = static_cast<double>(tdc);
        // (the one element whose interval holds tdc: the lane and slot that saw it)
        uint32_t mine = 0xFFFFFFFFu;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (key[t] != 0u && key[t] >= kx && static_cast<double>(E[t]) <= tt && tt < static_cast<double>(E[t] + q[t]))
            mine = key[t];
        const u64 hl = __ballot(mine != 0xFFFFFFFFu);
        ok = hl != 0ull;
        if (ok) {
          const uint32_t dk = __builtin_amdgcn_readlane(mine, __ffsll(static_cast<long long>(hl)) - 1);
          uint32_t fd, nd;
          u64 maboved, qd;
          group(dk, &fd, &nd, &maboved, &qd);
          u64 j = qd ? udiv53(tdc - maboved, qd) : 0ull;
          if (j >= nd) j = nd ? nd - 1 : 0;
          di = fd + static_cast<uint32_t>(j);
        }
      }
    }
    if (l == 0) {
      res[0] = ok ? 1u : 0u;
      res[1] = ck;
      res[2] = fc;
      res[3] = nc;
      res[4] = rr;
      res[5] = partial ? 1u : 0u;
      res[6] = di;
      res[7] = has_cut ? 1u : 0u;
      resq[0] = S;
      resq[1] = mabove;
      resq[2] = qc;
    }
  }
  __syncthreads();
  if (!res[0]) {
    __syncthreads();
    return false;
  }
  k.S = resq[0];
  if (res[7]) {
    k.has_cut = true;
    k.vc = val_of(res[1]);
    k.qc = resq[2];
    k.mabove_c = resq[1];
    k.r = res[4];
    k.partial = res[5] != 0u;
    if (!k.partial) k.x0 = k.vc;
  }
  const uint32_t fc = res[2];
  const int draw = a.out_probs ? 0 : c[res[6]].id;
  __syncthreads();
  // the id of the cutoff group's r-th member (resolve_idr's), from the list
  if (k.partial) {
    bool need = STATE || a.out_probs != nullptr;
    if (!need && p.draft >= 0 && p.draft < row.V && a.out_dprob) need = value_of(row, p.draft, &s.vslot) == k.vc;
    if (need) k.idr = c[fc + k.r - 1].id;
  }
  finish<STATE>(a, row, p, mz, k, draw, &s.vslot, r);
  return true;
}

// have_bitmap: the penalty pass left the penalised ids' bitmap at kBitmapOffset.
template <bool STATE, class Tin>
__device__ __forceinline__ void generic_row(const SampleArgs& a, Row<Tin> row, const RowParams& p, GenericSmem& g,
                                            FastSmem& f, int r, bool have_bitmap = false) {
  const int V = row.V;
  Search& s = g.srch;
  if (row.nexc > 0) {
    uint32_t* words = reinterpret_cast<uint32_t*>(&g) + kBitmapOffset;
    if (have_bitmap) row.bm = reinterpret_cast<const uint8_t*>(words);
    else build_bitmap(row, words);
  }
  // max (and first index of the max; NaN counts as the max); with top-k, in the same pass, a
  // histogram of the keys' top 13 bits
  const bool topk = p.K > 0 && p.K < V;  // (uniform)
  uint32_t* h13 = reinterpret_cast<uint32_t*>(&g) + kMatchOffset;
  constexpr int kTopBins = 8192;
  static_assert(kMatchOffset + kTopBins <= kChunk && kTopBins == 8 * kThreads, "top-k bins: eight per thread");
  if (topk) {
    for (int i = threadIdx.x; i < kTopBins; i += kThreads) h13[i] = 0;
    __syncthreads();
  }
  // The row's max: greedy rows (T <= 0) need its first index too, through ordered (key, id)
  // pairs; the others only its value, through fmax and a NaN flag (a NaN row's token, its first
  // NaN, is searched for afterwards), which costs a pass over an fp32 row a fraction of the
  // vector instructions
  const bool greedy = !(p.T > 0.0f);  // (uniform)
  u64 best = 0;
  float vmax = -INFINITY;
  uint32_t vnan = 0;
  // The bin of the kk-th largest key so far (thread t sums bins 8191 - 8t .. 8184 - 8t,
  // descending) to g.rdx.bk[0], the count above that bin to bk[1]; every thread calls, a
  // barrier publishes. (bk[0] keeps its value when fewer than kk keys were counted.)
  auto find_bin = [&](uint32_t kk) {
    uint32_t c8[8], s8 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c8[i] = h13[kTopBins - 1 - 8 * threadIdx.x - i];
      s8 += c8[i];
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan<uint32_t>(s8, g.rdx.hcnt, &tot);  // (hcnt: free until the descent)
    if (ex < kk && kk <= ex + s8) {
      uint32_t above = ex;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (above < kk && kk <= above + c8[i]) {
          g.rdx.bk[0] = static_cast<uint32_t>(kTopBins - 1 - 8 * threadIdx.x - i);
          g.rdx.bk[1] = above;
        }
        above += c8[i];
      }
    }
  };
  // fp32 rows with a small top-k: the first kStreamDepth stripes sample the row, and the bin of
  // their m-th largest key (m about twice the K-th's share of the sample) bounds the candidates
  // from below; the rest of the pass appends every element in that bin or above to a staging
  // list, which then holds the top-k candidates without a second pass over the row, and no
  // longer counts keys (checked below: the list must have kept all of them and hold the K-th
  // largest; its own histogram then gives the K-th largest's bin)
  constexpr int kStreamDepth = 2;
  Cand* stage = reinterpret_cast<Cand*>(reinterpret_cast<uint32_t*>(&g) + kMatchOffset + 2 * kCandCap);
  const bool stream = sizeof(Tin) == 4 && topk && p.K <= kStreamK && row.vec &&
                      row.V / kBlk / kThreads >= kStreamDepth;  // (uniform)
  uint32_t tau_bin = 0;
  auto first_pass = [&](auto greedy_c) {
    constexpr bool kGreedy = decltype(greedy_c)::value;
    auto visit_max = [&](float x, int id) {
      if constexpr (kGreedy) {
        const u64 kq = (static_cast<u64>(key_of(x)) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(id));
        best = kq > best ? kq : best;
      } else {
        vmax = fmaxf(vmax, x);
        vnan |= x != x ? 1u : 0u;
      }
    };
    auto visit = [&](float x, int id) {
      visit_max(x, id);
      if (topk) atomicAdd(&h13[key_of(x) >> 19], 1u);
    };
    if (stream) {
      if (threadIdx.x == 0) {
        g.rdx.bk[0] = 0;  // (the sample too small: every element is a candidate, the list overflows)
        g.rdx.bk[2] = 0;  // staged candidates
      }
      WholeBlock<Tin> q[kStreamDepth];
      uint32_t masked[kStreamDepth];
#pragma unroll
      for (int k = 0; k < kStreamDepth; ++k) {
        const int b = k * kThreads + threadIdx.x;
        q[k].load(row.p, b);
        masked[k] = row.bm ? row.bm[b] : 0u;
      }
      float v[kStreamDepth][kBlk];
#pragma unroll
      for (int k = 0; k < kStreamDepth; ++k) {
        q[k].values(v[k]);
#pragma unroll
        for (int i = 0; i < kBlk; ++i)
          if (!(masked[k] & (1u << i))) visit(v[k][i], (k * kThreads + static_cast<int>(threadIdx.x)) * kBlk + i);
      }
      __syncthreads();  // (the sample's histogram is complete)
      constexpr u64 kSample = static_cast<u64>(kStreamDepth) * kThreads * kBlk;
      find_bin(static_cast<uint32_t>((2ull * static_cast<u64>(p.K) * kSample + static_cast<u64>(V) - 1) / V) + 2u);
      __syncthreads();
      tau_bin = g.rdx.bk[0];
      // (x >= tau_x is key_of(x) >> 19 >= tau_bin for every non-NaN x: tau_x is the bin's
      // least value, or -inf below the least finite key's bin; a NaN row samples a point)
      const float tau_x = val_of(max(tau_bin << 19, key_of(-INFINITY)));
      auto append = [&](float x, int id) {
        const bool c = x >= tau_x;
        const u64 bal = __ballot(c);  // (one counter update per wave round)
        if (bal) {
          const int leader = __ffsll(static_cast<long long>(bal)) - 1;
          uint32_t at = 0;
          if (lane_id() == leader) at = atomicAdd(&g.rdx.bk[2], static_cast<uint32_t>(__popcll(bal)));
          at = __builtin_amdgcn_readlane(at, leader) +
               static_cast<uint32_t>(__popcll(bal & ((1ull << lane_id()) - 1ull)));
          if (c && at < static_cast<uint32_t>(kStreamCap)) stage[at] = Cand{x, id};
        }
      };
#pragma unroll
      for (int k = 0; k < kStreamDepth; ++k) {
#pragma unroll
        for (int i = 0; i < kBlk; ++i)
          if (!(masked[k] & (1u << i))) append(v[k][i], (k * kThreads + static_cast<int>(threadIdx.x)) * kBlk + i);
      }
      if (!kGreedy && tau_x > -INFINITY) {  // (uniform)
        // The rest of the row block by block: lanes without a bulk value enter as -inf (below
        // tau_x: never staged, never the max), the block's max by IEEE maximum (NaN when a value
        // is: the row's NaN test, after the loop), and the staging tests only where some lane's
        // block reaches tau_x -- in place of each element's branch, canonicalised fmax and NaN flag
        float mx = -INFINITY;
        for_each_block_ahead(row, [&](const float (&v)[kBlk], uint32_t out, int b) {
          float x[kBlk];
#pragma unroll
          for (int i = 0; i < kBlk; ++i) x[i] = out & (1u << i) ? -INFINITY : v[i];
          const float bx = max_of8(x);
          mx = __builtin_elementwise_maximum(mx, bx);
          if (__ballot(!(bx < tau_x))) {  // (uniform over the wave; a NaN block takes it too)
#pragma unroll
            for (int i = 0; i < kBlk; ++i) append(x[i], b * kBlk + i);
          }
        }, kStreamDepth);
        for (int e = threadIdx.x; e < row.nexc; e += kThreads) {
          visit_max(row.eval[e], row.eid[e]);
          append(row.eval[e], row.eid[e]);
        }
        vnan |= mx != mx ? 1u : 0u;
        vmax = fmaxf(vmax, mx);  // (mx: no NaN unless vnan)
      } else {
        for_each_ahead(row, [&](float x, int id) {
          visit_max(x, id);
          append(x, id);
        }, kStreamDepth);
      }
    } else {
      for_each(row, visit);
    }
  };
  if (greedy) first_pass(BoolC<true>{});
  else first_pass(BoolC<false>{});
  if (!greedy) best = static_cast<u64>(vnan ? 0xFFFFFFFFu : key_of(vmax)) << 32;
  best = block_max_u64(best, s.red64);  // (its barriers also end the histogram)
  const uint32_t nstage = stream ? g.rdx.bk[2] : 0u;
  const uint32_t mkey = static_cast<uint32_t>(best >> 32);
  int imax = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(best));
  if (!greedy && mkey == 0xFFFFFFFFu) imax = find_first(row, [&](float x, int) -> u64 { return x != x; }, 0ull, s);
  const float xmax = val_of(mkey);
  const float T = p.T;
  const float mz = xmax / T;
  Kept k;
  if (degenerate(row, p, mkey, imax, mz, s, k)) {
    finish<STATE>(a, row, p, mz, k, 0, &s.vslot, r);
    return;
  }
  const uint32_t lo_key = key_of(-INFINITY);
  uint32_t topbin = 0, ntop = kCandCap + 1u;  // the top-k candidates: bins >= topbin, ntop of them
  bool sorted = false;                          // (and sorted, when few)
  if (topk) {  // top-k: keep z >= kth largest z (sampler.py:53-55)
    // the bin of the K-th largest key (thread t sums bins 8191 - 8t .. 8184 - 8t, descending),
    // then the K'-th largest of that bin's elements, copied to LDS when they fit
    const uint32_t K = static_cast<uint32_t>(p.K);
    // (streamed: the histogram holds the sample only; the staged list's keys, or when it cannot
    // serve, another pass over the row's, replace it)
    const bool staged = stream && nstage >= K && nstage <= static_cast<uint32_t>(kStreamCap);  // (uniform)
    if (stream) {
      for (int i = threadIdx.x; i < kTopBins; i += kThreads) h13[i] = 0;
      __syncthreads();
      if (staged) {
        for (int i = threadIdx.x; i < static_cast<int>(nstage); i += kThreads) atomicAdd(&h13[key_of(stage[i].x) >> 19], 1u);
      } else {
        for_each(row, [&](float x, int) { atomicAdd(&h13[key_of(x) >> 19], 1u); });
      }
      __syncthreads();
    }
    find_bin(K);
    if (threadIdx.x == 0) g.rdx.ncand = 0;
    __syncthreads();  // (every read of the bins is done: the candidates go over them)
    // every element of that bin and the bins above (at most K - 1 of those): the K-th largest of
    // them is the row's; they hold every element >= x0 when x0 falls in those bins
    const uint32_t bin = g.rdx.bk[0];
    topbin = bin;
    Cand* cand = reinterpret_cast<Cand*>(h13);
    auto take = [&](float x, int id) {
      const bool c = (key_of(x) >> 19) >= bin;
      const u64 bal = __ballot(c);  // (one counter update per wave round)
      if (bal) {
        const int leader = __ffsll(static_cast<long long>(bal)) - 1;
        uint32_t at = 0;
        if (lane_id() == leader) at = atomicAdd(&g.rdx.ncand, static_cast<uint32_t>(__popcll(bal)));
        at = __builtin_amdgcn_readlane(at, leader) +
             static_cast<uint32_t>(__popcll(bal & ((1ull << lane_id()) - 1ull)));
        if (c && at < static_cast<uint32_t>(kCandCap)) cand[at] = Cand{x, id};
      }
    };
    // the staged list holds every element in bins >= tau_bin when it did not overflow, so the
    // K-th largest when it has at least K of them
    if (staged) {
      for (int i = threadIdx.x; i < static_cast<int>(nstage); i += kThreads) take(stage[i].x, stage[i].id);
    } else {
      for_each(row, take);
    }
    __syncthreads();
    const uint32_t nb = g.rdx.ncand;
    ntop = nb;
    sorted = nb <= static_cast<uint32_t>(kSortCap) && K <= nb;  // (uniform)
    if (sorted) sort_cands(cand, static_cast<int>(nb), cand + kCandCap);
    const CandList bl{cand, static_cast<int>(nb)};
    const uint32_t kkey = sorted ? key_of(cand[K - 1].x)
                          : nb <= static_cast<uint32_t>(kCandCap) ? radix_kth(row, &bl, K, g.rdx)
                                                                  : radix_kth(row, nullptr, K, g.rdx);
    if (threadIdx.x < kWave) {
      const float kz = val_of(kkey) / T;
      const uint32_t kx = bisect_key_wave(lo_key, kkey, [&](float x) { return x / T >= kz; });
      if (lane_id() == 0) g.rdx.bk[2] = kx;
    }
    __syncthreads();
    k.x0 = val_of(g.rdx.bk[2]);
    __syncthreads();
  }
  if (p.mp > 0.0f) {  // min-p: keep exp(z - max z) >= min_p
    if (threadIdx.x < kWave) {
      const double dmp = static_cast<double>(p.mp);
      const uint32_t kx = bisect_key_wave(lo_key, mkey, [&](float x) { return ptilde(x, T, mz) >= dmp; });
      if (lane_id() == 0) g.rdx.bk[3] = kx;
    }
    __syncthreads();
    const float xm = val_of(g.rdx.bk[3]);
    k.x0 = xm > k.x0 ? xm : k.x0;
    __syncthreads();
  }
  u64 S0 = 0;
  Cand* cand = reinterpret_cast<Cand*>(reinterpret_cast<uint32_t*>(&g) + kMatchOffset);
  static_assert(kMatchOffset + 2 * kCandCap <= kChunk, "the candidate list must fit");
  // (uniform) the top-k candidates already hold every element >= x0: no pass over the row
  const bool reuse = ntop <= static_cast<uint32_t>(kCandCap) && (key_of(k.x0) >> 19) >= topbin;
  const bool listable = k.x0 > -INFINITY;  // (uniform) a threshold: usually few candidates
  if (sorted && reuse && sorted_tail<STATE>(a, row, p, g, s, cand, static_cast<int>(ntop), mz, k, r)) return;
  if (reuse) {
    const float x0 = k.x0;
    for (int i = threadIdx.x; i < static_cast<int>(ntop); i += kThreads)
      if (cand[i].x >= x0) S0 += mass_q(ptilde(cand[i].x, T, mz));
    S0 = block_sum<u64>(S0, s.red64);
  } else {
  if (threadIdx.x == 0) g.rdx.ncand = 0;
  // (chunk masses of the elements >= x0: they lead the descents when the list does not fit)
  f.cmass[threadIdx.x] = 0;
  static_assert(kThreads == 1024, "one chunk per thread");
  __syncthreads();
  {
    const float x0 = k.x0;
    for_each(row, [&](float x, int id) {
      const bool c = x >= x0;
      if (c) {
        const u64 q = mass_q(ptilde(x, T, mz));
        S0 += q;
        atomicAdd(&f.cmass[(0xFFFFFFFFu - key_of(x)) >> 22], q);
      }
      // the candidates of this round of the wave: one counter update per wave
      const u64 bal = __ballot(listable && c);
      if (bal) {
        const int leader = __ffsll(static_cast<long long>(bal)) - 1;
        uint32_t at = 0;
        if (lane_id() == leader) at = atomicAdd(&g.rdx.ncand, static_cast<uint32_t>(__popcll(bal)));
        at = __builtin_amdgcn_readlane(at, leader) +
             static_cast<uint32_t>(__popcll(bal & ((1ull << lane_id()) - 1ull)));
        if (listable && c && at < static_cast<uint32_t>(kCandCap)) cand[at] = Cand{x, id};
      }
    });
    S0 = block_sum<u64>(S0, s.red64);  // (its barriers also publish the list)
  }
  }
  const uint32_t ncand = reuse ? ntop : g.rdx.ncand;
  const CandList cl{cand, static_cast<int>(ncand)};
  const CandList* list = (reuse || listable) && ncand <= static_cast<uint32_t>(kCandCap) ? &cl : nullptr;
  k.S = S0;
  if (p.tp < 1.0f) {  // top-p (sampler.py:57-64)
    const double P = static_cast<double>(p.tp) * static_cast<double>(S0);
    uint32_t nc;
    u64 massc, mabove;
    uint32_t ck;
    if (list) {
      ck = radix_mass(row, list, kCutoff, k.x0, T, mz, P, g.rdx, &nc, &massc, &mabove);
    } else {
      if (threadIdx.x < kWave) {
        u64 ab = 0;
        const int c = chunk_pick(f.cmass, kCutoff, P, &ab);
        if (lane_id() == 0) {
          g.rdx.bk[2] = static_cast<uint32_t>(c);
          g.rdx.bq[2] = ab;
        }
      }
      __syncthreads();
      const int c = static_cast<int>(g.rdx.bk[2]);
      const u64 ab = g.rdx.bq[2];
      __syncthreads();
      ck = c >= 0 ? radix_mass(row, nullptr, kCutoff, k.x0, T, mz, P, g.rdx, &nc, &massc, &mabove, 1023u - c, 10, ab)
                  : radix_mass(row, nullptr, kCutoff, k.x0, T, mz, P, g.rdx, &nc, &massc, &mabove);
    }
    k.has_cut = true;
    k.vc = val_of(ck);
    k.qc = nc ? massc / nc : 0ull;
    k.mabove_c = mabove;
    uint32_t rr = nc;
    if (k.qc > 0) {
      const double cr = ceil((P - static_cast<double>(mabove)) / static_cast<double>(k.qc));
      rr = cr < 1.0 ? 1u : (cr >= static_cast<double>(nc) ? nc : static_cast<uint32_t>(cr));
    }
    k.r = rr;
    k.partial = rr < nc;
    if (!k.partial) k.x0 = k.vc;
    k.S = mabove + static_cast<u64>(rr) * k.qc;
  }
  resolve_idr<STATE>(a, row, p, k, s);
  int draw = 0;
  if (!a.out_probs) {
    // the draw: descending value, ascending id within a value
    const u64 td = static_cast<u64>(static_cast<double>(p.u) * static_cast<double>(k.S));
    const u64 tdc = td < k.S ? td : k.S - 1;
    float vd;
    u64 j;
    if (k.has_cut && tdc >= k.mabove_c && k.qc > 0) {
      vd = k.vc;
      j = (tdc - k.mabove_c) / k.qc;
    } else {
      uint32_t nd;
      u64 massd, maboved;
      uint32_t dk;
      if (list) {
        dk = radix_mass(row, list, kCross, k.x0, T, mz, static_cast<double>(tdc), g.rdx, &nd, &massd, &maboved);
      } else {
        // (the chunk masses hold the elements >= the pre-cutoff x0; the draw lands above the
        // cutoff value here, where they are exact)
        if (threadIdx.x < kWave) {
          u64 ab = 0;
          const int c = chunk_pick(f.cmass, kCross, static_cast<double>(tdc), &ab);
          if (lane_id() == 0) {
            g.rdx.bk[2] = static_cast<uint32_t>(c);
            g.rdx.bq[2] = ab;
          }
        }
        __syncthreads();
        const int c = static_cast<int>(g.rdx.bk[2]);
        const u64 ab = g.rdx.bq[2];
        __syncthreads();
        dk = c >= 0 ? radix_mass(row, nullptr, kCross, k.x0, T, mz, static_cast<double>(tdc), g.rdx, &nd, &massd,
                                 &maboved, 1023u - c, 10, ab)
                    : radix_mass(row, nullptr, kCross, k.x0, T, mz, static_cast<double>(tdc), g.rdx, &nd, &massd,
                                 &maboved);
      }
      vd = val_of(dk);
      const u64 qd = nd ? massd / nd : 0ull;
      j = qd ? (tdc - maboved) / qd : 0ull;
      if (j >= nd) j = nd ? nd - 1 : 0;
    }
    // the j-th (ascending id) element equal to vd: from the candidate list when it holds at
    // most 64 of them (wave 0 ranks their ids), else from the row
    draw = -1;
    if (list) {
      if (threadIdx.x < kWave) {
        const int l = lane_id();
        uint32_t* ids = g.rdx.hcnt;  // (free: the descents are done)
        uint32_t cnt = 0;  // (uniform)
        for (int i0 = 0; i0 < list->n; i0 += kWave) {
          const int i = i0 + l;
          const bool m = i < list->n && list->c[i].x == vd;
          const u64 bal = __ballot(m);
          const uint32_t pos = cnt + static_cast<uint32_t>(__popcll(bal & ((1ull << l) - 1ull)));
          if (m && pos < static_cast<uint32_t>(kWave)) lds_poke(&ids[pos], static_cast<uint32_t>(list->c[i].id));
          cnt += static_cast<uint32_t>(__popcll(bal));
        }
        int res = -1;
        if (cnt <= static_cast<uint32_t>(kWave) && j < cnt) {
          wave_lds_sync();
          const uint32_t mine = static_cast<uint32_t>(l) < cnt ? lds_peek(&ids[l]) : 0xFFFFFFFFu;
          uint32_t rank = 0;
          for (uint32_t q = 0; q < cnt; ++q) rank += __builtin_amdgcn_readlane(mine, q) < mine ? 1u : 0u;
          const u64 hit = __ballot(static_cast<uint32_t>(l) < cnt && rank == j);
          if (hit) res = static_cast<int>(__builtin_amdgcn_readlane(mine, __ffsll(static_cast<long long>(hit)) - 1));
        }
        if (l == 0) g.rdx.bk[2] = static_cast<uint32_t>(res);
      }
      __syncthreads();
      draw = static_cast<int>(g.rdx.bk[2]);
      __syncthreads();
    }
    if (draw < 0) draw = find_first(row, [&](float x, int) -> u64 { return x == vd; }, j, s);
  }
  finish<STATE>(a, row, p, mz, k, draw, &s.vslot, r);
}

// ---- bf16 fast path: a 16-bit key histogram -----------------------------------------------------
// Ordered 16-bit key of raw bf16 bits (unsigned order = numeric order; -0.0 sits just below
// +0.0 and is folded onto it after the histogram is built).
__device__ __forceinline__ uint32_t ok16(uint32_t raw) {
  return raw ^ ((raw & 0x8000u) ? 0xFFFFu : 0x8000u);
}
__device__ __forceinline__ float val16(uint32_t ok) {
  const uint32_t raw = (ok & 0x8000u) ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
  return __uint_as_float(raw << 16);
}
__device__ __forceinline__ uint32_t hcount(const uint32_t* h, uint32_t ok) {
  return (h[ok >> 1] >> ((ok & 1u) << 4)) & 0xFFFFu;
}
// Chunk c holds keys 65535 - 64c - 63 .. 65535 - 64c; lane l of a chunk walk is key 65535-64c-l.
__device__ __forceinline__ int chunk_of16(uint32_t ok) { return static_cast<int>((65535u - ok) >> 6); }

enum WalkMode { kWalkCount = 0, kWalkCutoff = 1, kWalkCross = 2 };

struct WalkResult {
  uint32_t key;  // 32-bit ordered key of the value found
  uint32_t n;    // its group count (kept members)
  u64 q;         // mass of one member
  u64 above;     // count (kWalkCount) or mass strictly above it
  int ok;        // 0 if the chunk holds too many penalised values to resolve
};


// Resolve a value inside chunk c, by the 64 lanes of one wave and no workgroup barrier (the
// wave's LDS operations complete in order). `above` is the count or mass strictly above the
// chunk, `target` the 1-based rank (count) or the mass target. `ne` penalised values are in
// f.eid / f.eval. Every lane returns the result.
__device__ __forceinline__ WalkResult wave_walk(const uint32_t* hist, FastSmem& f, int ne, int c, int mode, u64 above,
                                                double target, float x0, float T, float mz) {
  const int l = lane_id();
  f.binc[l] = 0;
  f.binm[l] = 0;
  // the chunk's penalised values: first a list of their keys, compacted by ballot (a cheap pass
  // over all of them), then one list entry per lane: its mass, and the per-key counts and masses.
  // (A row that reaches a walk holds no NaN, so a value's key needs no NaN case; -0.0 takes
  // +0.0's key. The chunk's keys are klo .. klo + 2^22 - 1.)
  const bool has_pen = static_cast<uint32_t>(c) >= f.pchunk[0] && static_cast<uint32_t>(c) <= f.pchunk[1];
  const uint32_t klo = (65535u - 64u * static_cast<uint32_t>(c) - 63u) << 16;
  uint32_t nl = 0;
  // (four values a lane per step: 16-byte reads of eval, whose length is a multiple of 4)
  static_assert(kExcCap % 4 == 0, "eval is read four values at a time");
  for (int e0 = 0; has_pen && e0 < ne; e0 += 4 * kWave) {  // (uniform)
    const int e = e0 + 4 * l;
    const float4 x4 = e < ne ? *reinterpret_cast<const float4*>(&f.eval[e]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t bits = __float_as_uint(xs[j]);
      const uint32_t key =
          xs[j] == 0.0f ? 0x80000000u : bits ^ (static_cast<uint32_t>(static_cast<int32_t>(bits) >> 31) | 0x80000000u);
      const bool in = e + j < ne && key - klo < (1u << 22) && (mode == kWalkCount || xs[j] >= x0);
      const u64 b = __ballot(in);
      const uint32_t at = nl + lanes_below(b);
      if (in && at < static_cast<uint32_t>(kMaxL)) f.lkey[at] = key;
      nl += static_cast<uint32_t>(__popcll(b));
    }
  }
  WalkResult res;
  res.ok = nl <= static_cast<uint32_t>(kMaxL);
  wave_lds_sync();  // (the list's keys and the zeroed per-key sums are in)
  for (uint32_t i = static_cast<uint32_t>(l); res.ok && i < nl; i += kWave) {
    const uint32_t key = f.lkey[i];
    const u64 q = mode == kWalkCount ? 0ull : mass_q(ptilde(val_of(key), T, mz));
    f.lq[i] = q;
    const int lane = static_cast<int>(65535u - 64u * static_cast<uint32_t>(c) - (key >> 16));
    atomicAdd(&f.binc[lane], 1u);
    atomicAdd(&f.binm[lane], q);
  }
  wave_lds_sync();  // (the lanes' counts, masses and list masses are in)
  res.key = 0;
  res.n = 0;
  res.q = 0;
  res.above = 0;
  if (!res.ok) return res;
  const uint32_t K = 65535u - 64u * static_cast<uint32_t>(c) - l;
  const uint32_t cnt = hcount(hist, K);
  const float v = val16(K);
  const bool inb = mode == kWalkCount || v >= x0;
  const uint32_t cb = inb ? cnt : 0u;
  const u64 qb = (mode != kWalkCount && cb) ? mass_q(ptilde(v, T, mz)) : 0ull;
  const uint32_t bl = lds_peek(&f.binc[l]);
  const uint32_t cl = cb + bl;
  const u64 ml = (mode == kWalkCount ? static_cast<u64>(cl) : cb * qb + lds_peek(&f.binm[l]));
  const u64 inc = wave_incl_scan<u64>(ml);
  const u64 ab = above + inc - ml;  // strictly above this key
  bool hit;
  if (mode == kWalkCount) hit = static_cast<double>(ab) < target && target <= static_cast<double>(ab + ml);
  else if (mode == kWalkCutoff) hit = cl > 0 && static_cast<double>(ab) < target;
  else hit = ml > 0 && static_cast<double>(ab) <= target && target < static_cast<double>(ab + ml);
  const u64 hm = __ballot(hit);
  const int lw = hm ? (mode == kWalkCutoff ? 63 - __clzll(static_cast<long long>(hm))
                                           : __ffsll(static_cast<long long>(hm)) - 1)
                    : 0;
  const uint32_t cbw = __builtin_amdgcn_readlane(cb, lw);
  const u64 qbw = readlane64(qb, lw);
  const u64 abw = readlane64(ab, lw);
  const uint32_t nx = __builtin_amdgcn_readlane(bl, lw);
  const uint32_t Kw = 65535u - 64u * static_cast<uint32_t>(c) - lw;
  const uint32_t bkey = key_of(val16(Kw));
  if (nx == 0) {
    res.key = bkey;
    res.n = cbw;
    res.q = qbw;
    res.above = abw;
    return res;
  }
  // The key mixes its bf16 value with penalised values: its groups of equal values (the bulk
  // value's, with the penalised values equal to it, and the other penalised values') are resolved
  // by the whole wave. The list (at most 2 x 64 entries) is compacted to this key's entries; each
  // entry sums the weight of the entries above it and finds its equals (the first of them stands
  // for the group), and a wave max picks the hit group: the smallest value for the cutoff (hits
  // are the values whose weight above is below the target), the only one otherwise.
  static_assert(kMaxL <= 2 * kWave, "two list entries per lane");
  const bool counting = mode == kWalkCount;
  uint32_t ek[2];
  u64 eq[2];
  bool em[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t i = static_cast<uint32_t>(l + kWave * h);
    ek[h] = i < nl ? f.lkey[i] : 0u;
    eq[h] = i < nl ? f.lq[i] : 0ull;
    em[h] = i < nl && (ek[h] >> 16) == Kw;
  }
  const u64 b0 = __ballot(em[0]), b1 = __ballot(em[1]);
  const int n0 = __popcll(b0);
  const int n = n0 + __popcll(b1);
  wave_lds_sync();  // (every lane has read its entries before the list is overwritten)
  if (em[0]) {
    const int at = static_cast<int>(lanes_below(b0));
    f.lkey[at] = ek[0];
    f.lq[at] = eq[0];
  }
  if (em[1]) {
    const int at = n0 + static_cast<int>(lanes_below(b1));
    f.lkey[at] = ek[1];
    f.lq[at] = eq[1];
  }
  wave_lds_sync();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = l + kWave * h;
    ek[h] = i < n ? f.lkey[i] : 0u;
    eq[h] = i < n ? f.lq[i] : 0ull;
  }
  // (the loop's key and mass are uniform: the bulk value's weight above and its equal entries
  // are summed in scalar registers)
  const bool bulk = cbw > 0;
  u64 above_w[2] = {0ull, 0ull}, eq_m[2] = {0ull, 0ull}, above_b = abw;
  uint32_t eq_n[2] = {0u, 0u};
  bool first[2] = {true, true}, eq_b = false;
  for (int q = 0; q < n; ++q) {  // (uniform)
    const int ql = q & (kWave - 1);
    const uint32_t kq = __builtin_amdgcn_readlane(q < kWave ? ek[0] : ek[1], ql);
    const u64 qq = readlane64(q < kWave ? eq[0] : eq[1], ql);
    const u64 wq = counting ? 1ull : qq;
    if (kq > bkey) above_b += wq;
    if (kq == bkey) eq_b = true;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (kq > ek[h]) {
        above_w[h] += wq;
      } else if (kq == ek[h]) {
        eq_n[h] += 1u;
        eq_m[h] += qq;
        if (q < l + kWave * h) first[h] = false;
      }
    }
  }
  auto hits = [&](u64 acc, uint32_t gn, u64 gw) -> bool {
    if (mode == kWalkCount) return static_cast<double>(acc) < target && target <= static_cast<double>(acc + gw);
    if (mode == kWalkCutoff) return gn > 0 && static_cast<double>(acc) < target;
    return gw > 0 && static_cast<double>(acc) <= target && target < static_cast<double>(acc + gw);
  };
  // (the wave max's order: cutoff walks want the smallest key, the others the largest; 0 = none,
  // which no key in a walk takes: keys 0 and 0xFFFFFFFF are NaNs)
  auto order = [&](uint32_t key) -> uint32_t { return mode == kWalkCutoff ? ~key : key; };
  const u64 bw = counting ? static_cast<u64>(cbw) : static_cast<u64>(cbw) * qbw;
  uint32_t best = 0;
  u64 acc_h[2];
  uint32_t gn_h[2];
  bool hit_h[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const bool valid = l + kWave * h < n;
    const bool same = bulk && ek[h] == bkey;
    acc_h[h] = abw + above_w[h] + (bulk && bkey > ek[h] ? bw : 0ull);
    gn_h[h] = eq_n[h] + (same ? cbw : 0u);
    const u64 gm = eq_m[h] + (same ? static_cast<u64>(cbw) * qbw : 0ull);
    hit_h[h] = valid && first[h] && hits(acc_h[h], gn_h[h], counting ? static_cast<u64>(gn_h[h]) : gm);
    if (hit_h[h] && order(ek[h]) > best) best = order(ek[h]);
  }
  best = dpp::reduce(best, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
  // the bulk value's own group, when no penalised value equals it
  const bool hit_b = bulk && !eq_b && hits(above_b, cbw, bw);
  if (hit_b && order(bkey) > best) best = order(bkey);
  if (best == 0) {  // (no group hit: the bulk key, none kept)
    res.key = bkey;
    res.above = abw;
    return res;
  }
  if (hit_b && best == order(bkey)) {
    res.key = bkey;
    res.n = cbw;
    res.q = qbw;
    res.above = above_b;
    return res;
  }
  const u64 w0 = __ballot(hit_h[0] && order(ek[0]) == best), w1 = __ballot(hit_h[1] && order(ek[1]) == best);
  const bool hi = w0 == 0;
  const int at = __ffsll(static_cast<long long>(hi ? w1 : w0)) - 1;
  res.key = __builtin_amdgcn_readlane(hi ? ek[1] : ek[0], at);
  res.n = __builtin_amdgcn_readlane(hi ? gn_h[1] : gn_h[0], at);
  res.q = readlane64(hi ? eq[1] : eq[0], at);
  res.above = readlane64(hi ? acc_h[1] : acc_h[0], at);
  return res;
}

// Smallest key K in [lo, hi] with pred(val_of(K)) (pred(val_of(hi)) must hold; pred is false
// below the answer and true from it on), by the 64 lanes of one wave: 64 probes per round.
// `guess` is an estimate of the answer: the first round probes the 64 keys around it.
template <class P>
__device__ __forceinline__ uint32_t wave_bisect(uint32_t lo, uint32_t hi, uint32_t guess, P pred) {
  const uint32_t l = lane_id();
  if (lo < hi) {
    const uint32_t g = guess < lo ? lo : (guess > hi ? hi : guess);
    const uint32_t g0 = g - lo >= 32u ? g - 32u : lo;  // probes g0 .. g0 + 63, clamped to hi
    const u64 p64 = static_cast<u64>(g0) + l;
    const uint32_t probe = p64 < hi ? static_cast<uint32_t>(p64) : hi;
    const u64 hm = __ballot(pred(val_of(probe)));
    const int first = hm ? __ffsll(static_cast<long long>(hm)) - 1 : 64;
    // (first comes from a ballot: the same in every lane, so the lanes are read directly)
    if (first < 64) hi = __builtin_amdgcn_readlane(probe, first);
    if (first > 0) lo = __builtin_amdgcn_readlane(probe, first - 1) + 1;
    if (first == 0) lo = lo < hi ? lo : hi;
  }
  while (lo < hi) {
    // probes lo + step*(l+1) - 1 for l = 0..63 split [lo, hi] into 64 pieces
    const u64 span = static_cast<u64>(hi) - lo;
    const u64 step = (span + 63) / 64;
    const u64 probe64 = static_cast<u64>(lo) + step * (l + 1) - 1;
    const uint32_t probe = probe64 < hi ? static_cast<uint32_t>(probe64) : hi;
    const u64 hm = __ballot(pred(val_of(probe)));
    // the first probe that holds bounds the answer from above; the one before it from below
    const int first = hm ? __ffsll(static_cast<long long>(hm)) - 1 : 64;
    const uint32_t nhi = first < 64 ? __builtin_amdgcn_readlane(probe, first) : hi;
    const uint32_t nlo = first > 0 ? __builtin_amdgcn_readlane(probe, first - 1) + 1 : lo;
    lo = nlo;
    hi = nhi;
  }
  return hi;
}

// The id of the j-th (0-based, ascending id) token whose penalised value is vd: bulk positions
// holding vd that are not penalised, and penalised ids whose new value is vd.
// One pass writes, per 8-id block, the mask of its members into a byte cell (`cells`: cell b
// is block b, kThreads * cells_per(row) bytes of LDS, zeroed by the caller): unpenalised lanes
// whose bf16 value is vd (penalised lanes masked out by the position bitmap), then penalised ids
// whose new value is vd. Per-thread popcounts of consecutive cells and a scan find the block;
// its mask, the lane.
// Thread t holds the low bytes of the blocks it read in the histogram pass (t + m * kThreads,
// m < kLowBlocks: `low`, two words per block). A block whose low bytes hold none of vd's cannot
// hold a member; the others (the members' blocks and about 1/256 of the rest per distinct value
// of the row) are read again and matched in full, up to kProbe per thread at a time. Blocks
// m >= kLowBlocks (V > 155,648) are read again whole. `mxk` is the largest key the thread saw in
// the pass: a thread whose largest key is below vd's holds no member and reads nothing. Needs
// row.bm built when the row has penalised ids.
__device__ __forceinline__ int cells_per(const Row<uint16_t>& row) { return (row.nstripes + 3) & ~3; }

// Blocks per thread whose low bytes the histogram pass keeps in registers (2 words per block).
constexpr int kLowBlocks = 19;
constexpr int kProbe = 6;  // candidate blocks a thread reads at a time

// The low bytes of a block's eight bf16 values, elements 0-3 and 4-7 (v_perm_b32 picks bytes
// 0 and 2 of each word).
__device__ __forceinline__ uint32_t low4(uint32_t lo, uint32_t hi) { return __builtin_amdgcn_perm(hi, lo, 0x06040200u); }
// Bit 7 of byte i set when byte i of w is zero (and possibly for a byte above a zero byte): not
// 0 exactly when one of the four bytes of w is zero.
__device__ __forceinline__ uint32_t zero_bytes(uint32_t w) { return (w - 0x01010101u) & ~w & 0x80808080u; }

//
// Penalised ids need no position bitmap here: the bulk marking above marks every position whose
// original value is vd, penalised or not, and each thread then corrects the ids of its own
// penalised entries (`sl`: id << 13 | count, `og`: the original bf16 bits; f.eval holds the
// non-empty ones' new values at e0, e0 + estep, ...): a penalised id is a member exactly when
// its new value is vd.
__device__ __forceinline__ int select_member(const Row<uint16_t>& row, FastSmem& f, int ne, float vd, u64 j,
                                            uint8_t* cells, uint32_t mxk, const uint32_t (&low)[2 * kLowBlocks],
                                            const uint32_t (&sl)[4], const uint32_t (&og)[4], uint32_t e0,
                                            uint32_t estep) {
  const int tid = threadIdx.x;
  const uint32_t vb = __float_as_uint(vd);
  const bool bf = (vb & 0xFFFFu) == 0u;  // vd is a bf16 value: bulk tokens can hold it
  const uint32_t t16 = bf ? vb >> 16 : 0x10000u;  // 0x10000: matches no raw value
  const uint32_t t16b = vd == 0.0f ? (t16 ^ 0x8000u) : t16;  // -0.0 and +0.0 are one value
  const uint16_t* base = row.p;
  const int V = row.V;
  const int per = cells_per(row);  // cells per thread in the scan (a multiple of 4)
  uint32_t* cw = reinterpret_cast<uint32_t*>(cells);  // (zeroed by the caller, f.si[6] = -1)
  auto cell_or = [&](int id) {
    const int b = id / kBlk;
    atomicOr(&cw[b >> 2], 1u << (8 * (b & 3) + id % kBlk));
  };
  // The member lanes of an 8-element block: xor with the pattern zeroes the matching 16-bit
  // halves, v_pk_min_u16(x, 1) leaves 0 (match) or 1 per half, and three shifted ors gather the
  // halves of the 4 words into bits 0, 2, 4, 6 (low halves) and 16, 18, 20, 22 (high halves).
  // (The ones come through an opaque scalar register, or the compiler expands the min into
  // compares.)
  uint32_t ones_word;
  asm("s_mov_b32 %0, 0x10001" : "=s"(ones_word));
  const ushort2_t one2 = __builtin_bit_cast(ushort2_t, ones_word);
  auto nz2 = [&](uint32_t w, uint32_t pat) -> uint32_t {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(ushort2_t, w ^ pat), one2));
  };
  auto match1 = [&](uint4 w, uint32_t pat) -> uint32_t {
    const uint32_t a = nz2(w.x, pat) | (nz2(w.y, pat) << 2) | (nz2(w.z, pat) << 4) | (nz2(w.w, pat) << 6);
    return ~(a | (a >> 15)) & 0xFFu;
  };
  if (bf) {
    const uint32_t pat = t16 * 0x10001u, patb = t16b * 0x10001u;
    auto match8 = [&](uint4 w) -> uint32_t { return match1(w, pat) | (t16b != t16 ? match1(w, patb) : 0u); };
    const int nfull = row.vec ? V / kBlk : 0;
    const uint32_t ka = ok16(t16), kb = ok16(t16b);
    const bool cand = mxk >= (ka < kb ? ka : kb);
    // this thread's blocks tid + m * kThreads, m < nm
    const int nm = cand && tid < nfull ? (nfull - 1 - tid) / kThreads + 1 : 0;
    // (the low bytes of +0.0 and -0.0 are both 0: one pattern serves both)
    const uint32_t pat8 = (t16 & 0xFFu) * 0x01010101u;
    uint32_t todo = 0;  // bit m: block m's low bytes hold vd's (branch-free: 8 VALU per block)
    if (nm > 0) {
#pragma unroll
      for (int m = 0; m < kLowBlocks; ++m) {
        const uint32_t h = zero_bytes(low[2 * m] ^ pat8) | zero_bytes(low[2 * m + 1] ^ pat8);
        todo |= min(h, 1u) << m;
      }
      todo &= nm >= 32 ? 0xFFFFFFFFu : (1u << nm) - 1u;
    }
    // Up to kProbe candidate blocks per round, all requested before any is matched; a wave takes
    // as many slots as its lane with the most candidates (a lane without one rereads its first
    // block, unused).
    auto mark = [&](int b, uint4 w) {
      const uint32_t mask = match8(w);
      if (mask) cells[b] = static_cast<uint8_t>(mask);  // (block b belongs to this thread alone)
    };
    auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
    for (int round = 0; round < 4; ++round) {  // (19 blocks: at most 4 rounds of 6)
      const int slots = static_cast<int>(dpp::reduce(static_cast<uint32_t>(__popc(todo)), umax));  // (uniform)
      if (slots == 0) break;
      int mb[kProbe];
      uint4 w[kProbe];
#pragma unroll
      for (int c = 0; c < kProbe; ++c) {
        if (c < slots) {
          mb[c] = todo ? __ffs(todo) - 1 : -1;
          todo &= todo - 1u;
          w[c] = ld_block(base, mb[c] >= 0 ? tid + mb[c] * kThreads : min(tid, max(nfull - 1, 0)));
        }
      }
#pragma unroll
      for (int c = 0; c < kProbe; ++c)
        if (c < slots && mb[c] >= 0) mark(tid + mb[c] * kThreads, w[c]);
    }
    // blocks past the kept ones (V > 155,648), read again whole, four at a time
    if (__ballot(nm > kLowBlocks)) {  // (uniform)
      constexpr int D = 4;
      for (int m0 = kLowBlocks; __ballot(m0 < nm); m0 += D) {  // (uniform over the wave)
        uint4 q[D];
#pragma unroll
        for (int k = 0; k < D; ++k) q[k] = ld_block(base, min(tid + (m0 + k) * kThreads, max(nfull - 1, 0)));
#pragma unroll
        for (int k = 0; k < D; ++k)
          if (m0 + k < nm) mark(tid + (m0 + k) * kThreads, q[k]);
      }
    }
    lds_barrier();  // (the byte stores above land before the word atomics below)
    // the rest: a ragged tail, or every element of an unaligned row
    if (cand) {
      for (int i = nfull * kBlk + tid; i < V; i += kThreads) {
        const uint32_t raw = base[i];
        if (raw == t16 || raw == t16b) cell_or(i);
      }
    }
  }
  lds_barrier();  // (every bulk mark is in before the corrections)
  // this thread's penalised entries (at e0, e0 + estep, ... in the order of sl): members by
  // their new value, not their original one
  uint32_t e = e0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (sl[k] == kEmpty) continue;
    const int id = static_cast<int>(sl[k] >> 13);
    const uint32_t raw = og[k] & 0xFFFFu;
    const bool was = bf && (raw == t16 || raw == t16b);  // (the bulk marking set its bit)
    const bool is = f.eval[e] == vd;
    e += estep;
    if (was != is) {
      const int b = id / kBlk;
      const uint32_t bit = 1u << (8 * (b & 3) + id % kBlk);
      if (is) atomicOr(&cw[b >> 2], bit);
      else atomicAnd(&cw[b >> 2], ~bit);
    }
  }
  lds_barrier();
  // the cell holding the j-th member: per-thread member counts of `per` consecutive cells (one
  // popcount per 4 cells), then a scan
  // (the thread's cells stay in registers: the thread holding the j-th member finds it there)
  const int c0 = tid * per;
  constexpr int kCellWords = 8;  // per <= 32 (the caller's bound on cells_per)
  uint32_t cv[kCellWords];
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < kCellWords; ++i) {
    cv[i] = 4 * i < per ? cw[(c0 >> 2) + i] : 0u;
    mine += __popc(cv[i]);
  }
  uint32_t total;
  const uint32_t before = block_excl_scan<uint32_t>(mine, f.red32, &total);
  if (total > 0 && j < total && before <= j && j < before + mine) {
    // the word, then the cell (byte) within it, then the lane within the cell
    uint32_t r = static_cast<uint32_t>(j - before), word = 0;
    int wi = -1;
#pragma unroll
    for (int i = 0; i < kCellWords; ++i) {
      const uint32_t n = __popc(cv[i]);
      if (wi < 0) {
        if (r < n) {
          wi = i;
          word = cv[i];
        } else {
          r -= n;
        }
      }
    }
    int bi = -1;
    uint32_t mask = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t m8 = (word >> (8 * b)) & 0xFFu;
      const uint32_t n = __popc(m8);
      if (bi < 0) {
        if (r < n) {
          bi = b;
          mask = m8;
        } else {
          r -= n;
        }
      }
    }
    for (; r > 0; --r) mask &= mask - 1;
    f.si[6] = (c0 + 4 * wi + bi) * kBlk + __ffs(mask) - 1;
  }
  lds_barrier();
  return f.si[6];  // (a caller that searches again resets f.si[6] only after another barrier)
}

// (merge mode) The id of the j-th (0-based, ascending id) token whose penalised value is v, or
// -1. Each slice's count of members comes from its record (the bulk count of v's key; of both
// zero keys when v is 0), minus its penalised ids whose original value is v, plus its penalised
// ids whose new value is v; the slice holding the j-th member is then searched alone, as a row
// of its own. `scratch` is LDS past the position bitmap (kMaxSlices + 2 kExcCap + 4 words);
// needs row.bm built when the row has penalised ids.
__device__ __forceinline__ int split_find(const SampleArgs& a, const Row<uint16_t>& row, FastSmem& f, int ne,
                                          float v, u64 j, Search& srch, uint32_t* scratch, const uint8_t* recs) {
  const int tid = threadIdx.x;
  const int G = a.G;
  uint32_t* cnt = scratch;
  int32_t* xid = reinterpret_cast<int32_t*>(scratch + kMaxSlices);
  float* xval = reinterpret_cast<float*>(scratch + kMaxSlices + kExcCap);
  uint32_t* misc = scratch + kMaxSlices + 2 * kExcCap;  // listed ids, the slice, the index in it
  const uint32_t vb = __float_as_uint(v);
  const bool bf = (vb & 0xFFFFu) == 0u;  // bulk tokens can hold v
  const int nfull = row.V / kBlk;
  if (tid < G) {
    uint32_t c = 0;
    if (bf) {
      const uint32_t k1 = ok16(vb >> 16);
      const uint32_t k2 = v == 0.0f ? ok16((vb >> 16) ^ 0x8000u) : k1;
      const uint8_t* rec = recs + static_cast<size_t>(tid) * kSliceRecord;
      for (int t = 0; t < (k2 != k1 ? 2 : 1); ++t) {
        const uint32_t key = t ? k2 : k1;
        const uint32_t ch = (65535u - key) >> 6;
        const uint32_t e = ld_dev<uint16_t>(reinterpret_cast<const uint16_t*>(rec + kSliceEmap) + ch);
        if (e != kNoEntry) {
          const uint32_t w0 = 32768u - 32u * ch - 32u;  // the chunk's first histogram word
          const uint32_t word = ld_dev<uint32_t>(reinterpret_cast<const uint32_t*>(rec + kSliceData) + 32u * e + ((key >> 1) - w0));
          c += (word >> ((key & 1u) << 4)) & 0xFFFFu;
        }
      }
    }
    cnt[tid] = c;
  }
  if (tid == 0) misc[0] = 0;
  lds_barrier();
  auto slice_of = [&](int id) {  // the last g with slice_begin(g) <= id's block
    const int64_t b = id / kBlk;
    const int g = static_cast<int>(((b + 1) * G + nfull - 1) / nfull) - 1;
    return g < G - 1 ? g : G - 1;
  };
  for (int e = tid; e < ne; e += kThreads) {
    const int id = f.eid[e];
    const int g = slice_of(id);
    if (bf && bf16_to_f32(ld_global(row.p + id)) == v) atomicSub(&cnt[g], 1u);
    if (f.eval[e] == v) atomicAdd(&cnt[g], 1u);
  }
  lds_barrier();
  if (tid < kWave) {
    const u64 c = tid < G ? cnt[tid] : 0u;
    const u64 inc = wave_incl_scan<u64>(c);
    const bool hit = c > 0 && inc - c <= j && j < inc;
    const u64 hm = __ballot(hit);
    if (tid == 0) misc[1] = hm ? static_cast<uint32_t>(__ffsll(static_cast<long long>(hm)) - 1) : 0xFFFFFFFFu;
    if (hit) misc[2] = static_cast<uint32_t>(j - (inc - c));
  }
  lds_barrier();
  const uint32_t gs = misc[1];
  if (gs == 0xFFFFFFFFu) return -1;  // (uniform)
  const u64 jj = misc[2];
  const int b0 = slice_begin(nfull, G, static_cast<int>(gs));
  const int s0 = b0 * kBlk;
  const int s1 = static_cast<int>(gs) == G - 1 ? row.V : slice_begin(nfull, G, static_cast<int>(gs) + 1) * kBlk;
  for (int e = tid; e < ne; e += kThreads) {
    const int id = f.eid[e];
    if (id >= s0 && id < s1) {
      const uint32_t i = atomicAdd(&misc[0], 1u);
      xid[i] = id - s0;
      xval[i] = f.eval[e];
    }
  }
  lds_barrier();
  Row<uint16_t> sr = row;
  sr.p = row.p + s0;
  sr.V = s1 - s0;
  sr.nblk = (sr.V + kBlk - 1) / kBlk;
  sr.nstripes = (sr.nblk + kThreads - 1) / kThreads;
  sr.bm = row.bm ? row.bm + b0 : nullptr;
  sr.eid = xid;
  sr.eval = xval;
  sr.nexc = static_cast<int>(misc[0]);
  const int res = find_first(sr, [&](float x, int) -> u64 { return x == v ? 1ull : 0ull; }, jj, srch);
  return res < 0 ? -1 : res + s0;
}

// The bf16 fast path (every temperature: T <= 0 is greedy). Returns false (before writing any
// output) when the row needs the generic path: a history longer than kFastMaxL or with more
// than kExcCap distinct ids, a key count past 65535, or a chunk with more than kMaxL penalised
// values. `srch` and the match list alias
// `hist`: they are used only once the histogram is no longer read.
//
// With PEN the row's history is counted here, between the first rounds of the histogram pass,
// and the penalised ids' original values are gathered while the pass streams the row; the
// penalised ids and values end in f.eid / f.eval.
//
// `pw` is parameter word tid of the row (threads below kParamWords), loaded by the caller; the
// parameters reach f.prm (read through `p`) once the row's first loads are issued.
//
// Loads here sit outside divergent branches (a lane past the end rereads a valid block whose
// data it ignores): a load inside one needs a copy at the join, and that copy waits for every
// load in flight.
// SPLIT: the workgroup takes one slice of the row (split.cuh): it builds the slice's histogram
// and record and returns true unless it is the row's last slice to arrive, which adds the other
// slices' records to its histogram and finishes the row; the drawn member is found by
// split_find. `r` is the row.
template <bool PEN, bool STATE, bool SPLIT = false>
__device__ __forceinline__ bool fast_row(const SampleArgs& a, Row<uint16_t> row, const RowParams& p, uint32_t* hist,
                                         FastSmem& f, Search& srch, uint32_t pw, int r) {
  const int tid = threadIdx.x;
  const int V = row.V;
  // ---- 1. histogram of every key, then the penalised tokens' original keys taken out ----------
  // (u16 halves of a word wrap and borrow exactly: only the final counts must stay below 2^16)
  const uint16_t* base = row.p;
  const int nfull = row.vec ? V / kBlk : 0;  // blocks read as one 16-byte load
  // A rolling prefetch: slot k of d holds block tid + (D * round + k) * kThreads and is reloaded
  // for the next round as soon as it is consumed (into the same registers: loading before the
  // old value is consumed would need a copy at the loop's end, which waits for every load).
  // (A row with no full block loads a constant block instead, unused: loads issued on one branch
  // only would make the first wait for the parameters wait for every load in flight.)
  constexpr int D = 4;
  uint4 d[D];
  if constexpr (!SPLIT) {
    const uint16_t* src = nfull > 0 ? base : g_unused_block;
#pragma unroll
    for (int k = 0; k < D; ++k) d[k] = ld_block(src, min(tid + k * kThreads, max(nfull - 1, 0)));
  }
  // (split rows) this workgroup's slice of the row and the row's slice records
  uint8_t* recs = SPLIT ? a.slices + static_cast<size_t>(r) * a.G * kSliceRecord : nullptr;
  const int gown = SPLIT ? static_cast<int>(blockIdx.x) / a.nrows : 0;
  if (tid < kParamWords) reinterpret_cast<uint32_t*>(&f.prm)[tid] = pw;
  uint32_t* htab = fast_htab(f);
  for (int i = tid; i < kChunk / 4; i += kThreads) reinterpret_cast<uint4*>(hist)[i] = make_uint4(0, 0, 0, 0);
  // (uniform) the history is counted in a presence bitmap, else in the hash table
  const bool presence = PEN && V <= kPresMaxV;
  const int nw64 = (V + 63) / 64;
  if (presence) {
    // the counts and the bitmap
    for (int i = tid; i < (kPresBits + 2 * nw64 + 3) / 4; i += kThreads)
      reinterpret_cast<uint4*>(htab)[i] = make_uint4(0, 0, 0, 0);
  } else {
    reinterpret_cast<uint4*>(htab)[tid] = make_uint4(kEmpty, kEmpty, kEmpty, kEmpty);
  }
  static_assert(kFastSlots == 4 * kThreads && kPresBits % 4 == 0, "one uint4 of slots per thread");
  if (tid == 0) f.hfail = 0;
  if (tid == 0) {
    f.pchunk[0] = kThreads;
    f.pchunk[1] = 0;
  }
  lds_barrier();
  const float T = uniform_f(p.T);
  const int L = PEN ? p.h1 - p.h0 : 0;
  const bool on = PEN && L > 0 && (p.rep != 1.0f || p.pres != 0.0f || p.freq != 0.0f);
  const bool pen = on && L <= kFastMaxL;  // a longer history is counted by the generic path
  // history positions tid + k * kThreads (clamped to the last). With PEN they are loaded whether
  // or not the row counts a history (a row that does not reads the batch's first history id and
  // ignores it): loads issued on one branch only make the first use of the row's blocks wait for
  // every load.
  uint32_t hid[kFastHistPer];
  if constexpr (PEN) {
    const int32_t* h = a.pen.hist + (pen ? p.h0 : 0);
    const int hl = pen ? L - 1 : 0;
#pragma unroll
    for (int k = 0; k < kFastHistPer; ++k) hid[k] = static_cast<uint32_t>(ld_global(h + min(tid + k * kThreads, hl)));
  }

  // mx2: the largest key this thread has seen, per 16-bit half (the member search skips the
  // threads whose largest key is below the value it looks for)
  ushort2_t mx2 = ushort2_t{0, 0};
  auto add2 = [&](uint32_t w) {
    // ordered keys of both halves at once: xor with (sign ? 0xFFFF : 0x8000)
    const uint32_t k2 = ok16x2(w);
    const uint32_t klo = k2 & 0xFFFFu, khi = k2 >> 16;
    atomicAdd(&hist[klo >> 1], 1u << ((klo & 1u) << 4));
    atomicAdd(&hist[khi >> 1], 1u << ((khi & 1u) << 4));
    mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(ushort2_t, k2));
  };
  // the history: after round 0 each thread inserts its ids; after round 1 the table is
  // compacted (thread t keeps slots 4t .. 4t + 3 in sl) and the ids' original values are
  // loaded, in flight through the remaining rounds. (Rounds 0 and 1 are peeled off the loop:
  // a value defined inside a loop and carried round it takes a copy that waits for every load
  // in flight.)
  uint32_t sl[4] = {kEmpty, kEmpty, kEmpty, kEmpty};
  uint32_t e0 = 0, nexc = 0;
  const int rounds = SPLIT ? 1 : (nfull + D * kThreads - 1) / (D * kThreads);  // (uniform)
  uint32_t low[2 * kLowBlocks];  // the low bytes of this thread's blocks, for the member search
  auto round = [&](int it) {
    if constexpr (SPLIT) {
      // (the row's last slice) the other slices' records into the histogram
      slice_merge(recs, a.G, gown, hist, f.lkey);
      return;
    }
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const int b = tid + (it * D + k) * kThreads;
      if (b < nfull) {
        add2(d[k].x);
        add2(d[k].y);
        add2(d[k].z);
        add2(d[k].w);
      }
      if (it * D + k < kLowBlocks) {  // (a constant test at every peeled round, false in the loop)
        low[2 * (it * D + k)] = low4(d[k].x, d[k].y);
        low[2 * (it * D + k) + 1] = low4(d[k].z, d[k].w);
      }
      d[k] = ld_block(base, min(b + D * kThreads, nfull - 1));
    }
  };
  if constexpr (SPLIT) {
    // this slice's keys, its record, and its arrival: only the row's last slice goes on
    slice_hist(base, V, a.G, gown, hist);
    lds_barrier();
    slice_record(hist, recs + static_cast<size_t>(gown) * kSliceRecord, f.red32);
    if (!slice_arrive(a.arrive + r, a.epoch, a.G, &f.si[7])) return true;  // (uniform)
  }
  if (rounds > 0) round(0);
  // The presence path's four steps follow rounds 0 .. 3, each while the next round's blocks
  // arrive: the bits and their prefix; ranks and counts; the ids in rank order; each thread's two
  // entries (ranks tid and tid + kThreads), whose original values are then loaded.
  uint32_t estep = 1;  // list positions of this thread's entries: e0, e0 + estep, ...
  uint32_t* bm32 = htab + kPresBits;
  const u64* bm64 = reinterpret_cast<const u64*>(bm32);
  uint16_t* pre16 = reinterpret_cast<uint16_t*>(bm32 + 2 * nw64);
  auto valid = [&](int k) { return tid + k * kThreads < L && hid[k] < static_cast<uint32_t>(V); };  // (ids outside [0, V) are skipped)
  u64 bw[kPresPer] = {0, 0, 0};
  uint32_t pw3[kPresPer] = {0, 0, 0};
  static_assert(kPresPer == 3, "three words per thread");
  if (pen && presence) {
#pragma unroll
    for (int k = 0; k < kFastHistPer; ++k)
      if (valid(k)) atomicOr(&bm32[hid[k] >> 5], 1u << (hid[k] & 31u));
    lds_barrier();
#pragma unroll
    for (int i = 0; i < kPresPer; ++i) {
      const int w = kPresPer * tid + i;
      bw[i] = w < nw64 ? bm64[w] : 0ull;
    }
    const uint32_t n0 = __popcll(bw[0]), n1 = __popcll(bw[1]), n2 = __popcll(bw[2]);
    e0 = block_excl_scan<uint32_t>(n0 + n1 + n2, f.red32, &nexc);
    if (nexc > static_cast<uint32_t>(kExcCap)) return false;  // (uniform)
    pw3[0] = e0;
    pw3[1] = e0 + n0;
    pw3[2] = e0 + n0 + n1;
#pragma unroll
    for (int i = 0; i < kPresPer; ++i)
      if (kPresPer * tid + i < nw64) pre16[kPresPer * tid + i] = static_cast<uint16_t>(pw3[i]);
  }
  if (pen && !presence) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < kFastHistPer; ++k)
      if (valid(k)) ok = fast_insert(htab, hid[k]) && ok;
    if (!ok) f.hfail = 1;
  }
  if (rounds > 1) round(1);
  if (pen && presence) {
    lds_barrier();
#pragma unroll
    for (int k = 0; k < kFastHistPer; ++k) {
      if (!valid(k)) continue;
      const uint32_t w = hid[k] >> 6;
      const uint32_t rank = pre16[w] + static_cast<uint32_t>(__popcll(bm64[w] & ((1ull << (hid[k] & 63u)) - 1ull)));
      atomicAdd(&htab[rank >> 1], 1u << ((rank & 1u) << 4));
    }
  }
  if (pen && !presence) {
    lds_barrier();
    const uint4 s4 = reinterpret_cast<const uint4*>(htab)[tid];
    sl[0] = s4.x;
    sl[1] = s4.y;
    sl[2] = s4.z;
    sl[3] = s4.w;
    uint32_t n = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) n += sl[k] != kEmpty ? 1u : 0u;
    e0 = block_excl_scan<uint32_t>(n, f.red32, &nexc);  // (its barriers end every read of htab)
    if (f.hfail || nexc > static_cast<uint32_t>(kExcCap)) return false;
  }
  if (on && !pen) return false;
  if (rounds > 2) round(2);
  uint32_t* ids = htab + kPresBits;
  if (pen && presence) {
    lds_barrier();  // (every read of the bitmap and the prefix is done: the ids go over them)
#pragma unroll
    for (int i = 0; i < kPresPer; ++i) {
      uint32_t rk = pw3[i];
      for (u64 m = bw[i]; m; m &= m - 1) ids[rk++] = 64u * (kPresPer * tid + i) + static_cast<uint32_t>(__builtin_ctzll(m));
    }
  }
  if (rounds > 3) round(3);
  if (pen && presence) {
    lds_barrier();
    const uint16_t* cnt16 = reinterpret_cast<const uint16_t*>(htab);
    const uint32_t ra = tid, rb = tid + kThreads;
    sl[0] = ra < nexc ? (ids[ra] << 13) | cnt16[ra] : kEmpty;  // (id << 13 | count)
    sl[1] = rb < nexc ? (ids[rb] << 13) | cnt16[rb] : kEmpty;
    e0 = tid;
    estep = kThreads;
  }
  uint32_t og[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) og[k] = ld_global(base + (sl[k] != kEmpty ? sl[k] >> 13 : 0u));
  static_assert(kLowBlocks <= 5 * D, "the blocks whose low bytes are kept are read in the peeled rounds");
  // (round 4 is peeled too: the first use of its blocks then waits for them alone, not for the
  // original values just requested, as a wait at a loop's head would)
  if (rounds > 4) round(4);
  for (int it = 5; it < rounds; ++it) round(it);
  // the rest: a ragged tail, or every element of an unaligned row
  uint32_t mxk = mx2.x > mx2.y ? mx2.x : mx2.y;
  for (int i = nfull * kBlk + tid; !SPLIT && i < V; i += kThreads) {  // (split rows: the last slice's)
    const uint32_t ko = ok16(base[i]);
    atomicAdd(&hist[ko >> 1], 1u << ((ko & 1u) << 4));
    mxk = ko > mxk ? ko : mxk;
  }
  // the penalised ids: original keys out of the histogram, penalised values into the list
  if (pen) {
    uint32_t e = e0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (sl[k] == kEmpty) continue;  // (the presence path fills sl[0] and sl[1] only)
      const uint32_t ko = ok16(og[k]);
      atomicAdd(&hist[ko >> 1], 0u - (1u << ((ko & 1u) << 4)));
      f.eid[e] = static_cast<int32_t>(sl[k] >> 13);
      f.eval[e] = apply_penalty(bf16_to_f32(static_cast<uint16_t>(og[k])), static_cast<int>(sl[k] & 0x1FFFu),
                                p.rep, p.pres, p.freq);
      e += estep;
    }
  }
  const int ne = static_cast<int>(nexc);
  row.nexc = ne;
  lds_barrier();
  // fold -0.0 (key 0x7FFF, high half of word 0x3FFF) onto +0.0 (key 0x8000, low half of 0x4000)
  if (tid == 0) {
    const uint32_t neg0 = hist[0x3FFF] >> 16;
    const uint32_t pos0 = hist[0x4000] & 0xFFFFu;
    f.si[1] = 0;
    if (neg0) {
      if (pos0 + neg0 > 0xFFFFu) f.si[1] = 1;  // would overflow: generic path
      hist[0x3FFF] &= 0xFFFFu;
      hist[0x4000] += neg0;
    }
  }
  lds_barrier();
  // The rest alternates parallel phases (all threads, one barrier each) with decisions taken by
  // wave 0 alone (no workgroup barrier inside), which it publishes in f.plan.
  // ---- 2. [all] per-chunk counts, NaNs, the top chunk, the penalised max ---------------------
  {
    uint32_t cnt = 0, nan = 0;
    const int w0 = 32768 - 32 * tid - 32;  // the chunk's 32 words: keys 2*w0 .. 2*w0 + 63
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int piece = (s + tid) & 7;  // rotate so a wave's 16-byte reads spread over the banks
      const uint4 q4 = *reinterpret_cast<const uint4*>(&hist[w0 + 4 * piece]);
      // lo + hi of each word in one v_dot2_u32_u16
      cnt = __builtin_amdgcn_udot2(__builtin_bit_cast(ushort2_t, q4.x), ones2(), cnt, false);
      cnt = __builtin_amdgcn_udot2(__builtin_bit_cast(ushort2_t, q4.y), ones2(), cnt, false);
      cnt = __builtin_amdgcn_udot2(__builtin_bit_cast(ushort2_t, q4.z), ones2(), cnt, false);
      cnt = __builtin_amdgcn_udot2(__builtin_bit_cast(ushort2_t, q4.w), ones2(), cnt, false);
    }
    // NaN keys: all of chunks 0 and 1023 (keys >= 0xFFC0, <= 0x003F), and chunks 1 and 1022
    // but for +inf (0xFF80) and -inf (0x007F)
    if (tid == 0 || tid == 1023) nan = cnt;
    if (tid == 1) nan = cnt - hcount(hist, 0xFF80u);
    if (tid == 1022) nan = cnt - hcount(hist, 0x007Fu);
    f.ccnt[tid] = cnt;
    f.cmass[tid] = 0;
    // penalised values: their max and NaNs
    uint32_t emax = 0, emin = 0xFFFFFFFFu;
    for (int e = tid; e < ne; e += kThreads) {
      const uint32_t key = key_of(f.eval[e]);
      if (key == 0xFFFFFFFFu) ++nan;
      emax = key > emax ? key : emax;
      emin = key < emin ? key : emin;
    }
    const uint32_t code = cnt ? static_cast<uint32_t>(1024 - tid) : 0u;  // higher = larger keys
    auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
    const uint4 wpart = make_uint4(wave_sum<uint32_t>(cnt), wave_sum<uint32_t>(nan), dpp::reduce(code, umax),
                                   dpp::reduce(emax, umax));
    // the penalised values' chunk range (wave_walk skips the list outside it)
    const uint32_t wmin = ~dpp::reduce(~emin, umax);
    if (lane_id() == 0) {
      f.wp[tid / kWave] = wpart;
      if (wpart.w) {
        atomicMin(&f.pchunk[0], static_cast<uint32_t>(chunk_of16(wpart.w >> 16)));
        atomicMax(&f.pchunk[1], static_cast<uint32_t>(chunk_of16(wmin >> 16)));
      }
    }
  }
  lds_barrier();
  // ---- 3. [wave 0] totals, the max, point rows, top-k and min-p thresholds -----------------
  const uint32_t lo_key = key_of(-INFINITY);
  if (tid < kWave) {
    const int l = tid;
    const uint4 wq = l < kWaves ? f.wp[l] : make_uint4(0, 0, 0, 0);
    auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
    const uint32_t total = wave_sum<uint32_t>(wq.x);
    const uint32_t nnan = wave_sum<uint32_t>(wq.y);
    const uint32_t cm = dpp::reduce(wq.z, umax);
    const uint32_t em = dpp::reduce(wq.w, umax);
    int status = kPlanFast;
    uint32_t mkey = 0;
    float x0 = -INFINITY, mz = 0.0f;
    if (f.si[1] || total != static_cast<uint32_t>(V - ne)) {
      status = kPlanGeneric;  // a key count past 65535
    } else {
      // the bulk max: the top populated key of the top populated chunk
      uint32_t mk = 0;
      if (cm) {
        const uint32_t top = 65535u - 64u * (1024u - cm);
        const u64 hb = __ballot(hcount(hist, top - l) != 0);
        if (hb) mk = key_of(val16(top - (__ffsll(static_cast<long long>(hb)) - 1)));
      }
      mkey = em > mk ? em : mk;
      const float xmax = val_of(mkey);
      mz = xmax / T;
      if (nnan || !(T > 0.0f) || mz != mz || mz == INFINITY || mz == -INFINITY) {
        status = kPlanPoint;
      } else {
        // top-k: the K-th largest value's chunk (penalised values join their chunks' counts),
        // its value, then the smallest x with fl32(x / T) >= its z
        if (p.K > 0 && p.K < V) {
          for (int e = l; e < ne; e += kWave) atomicAdd(&f.ccnt[chunk_of16(key_of(f.eval[e]) >> 16)], 1u);
          wave_lds_sync();
          uint32_t cc[16];
          uint32_t sum = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint4 v4 = *reinterpret_cast<const uint4*>(&f.ccnt[16 * l + 4 * q]);
            cc[4 * q] = v4.x;
            cc[4 * q + 1] = v4.y;
            cc[4 * q + 2] = v4.z;
            cc[4 * q + 3] = v4.w;
            sum += v4.x + v4.y + v4.z + v4.w;
          }
          uint32_t ex = wave_incl_scan<uint32_t>(sum) - sum;
          const uint32_t Kq = static_cast<uint32_t>(p.K);
          int ck = -1;
          uint32_t cab = 0;
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            if (ck < 0 && ex < Kq && Kq <= ex + cc[q]) {
              ck = 16 * l + q;
              cab = ex;
            }
            ex += cc[q];
          }
          const u64 hm = __ballot(ck >= 0);
          if (!hm) {
            status = kPlanGeneric;
          } else {
            const int lw = __ffsll(static_cast<long long>(hm)) - 1;
            ck = __builtin_amdgcn_readlane(ck, lw);
            cab = __builtin_amdgcn_readlane(cab, lw);
            const WalkResult wr = wave_walk(hist, f, ne, ck, kWalkCount, cab, static_cast<double>(p.K), -INFINITY, T, mz);
            if (!wr.ok) {
              status = kPlanGeneric;
            } else {
              const float kz = val_of(wr.key) / T;
              x0 = val_of(wave_bisect(lo_key, wr.key, key_of(kz * T), [&](float x) { return x / T >= kz; }));
            }
          }
        }
        // min-p: the smallest x with exp(fl32(x / T) - max z) >= min_p
        if (status == kPlanFast && p.mp > 0.0f) {
          const double dmp = static_cast<double>(p.mp);
          // (only a starting point for the bisection, which tests every step exactly)
          const float guess = T * (mz + __logf(p.mp));
          const float xm = val_of(wave_bisect(lo_key, mkey, key_of(guess), [&](float x) { return ptilde(x, T, mz) >= dmp; }));
          x0 = xm > x0 ? xm : x0;
        }
      }
    }
    if (l == 0) {
      f.plan.status = status;
      f.plan.mkey = mkey;
      f.plan.nnan = nnan;
      f.plan.x0 = x0;
      f.plan.mz = mz;
    }
  }
  lds_barrier();
  const int status = f.plan.status;
  if (status == kPlanGeneric) return false;
  const uint32_t mkey = uniform_u(f.plan.mkey);
  const float mz = uniform_f(f.plan.mz);
  Kept k;
  // The histogram is dead from here on: the id searches use its memory. The penalised ids'
  // position bitmap is built only for a search that passes over the row (find_first, split
  // rows' slice search, probabilities): the member search corrects penalised ids itself.
  auto need_bitmap = [&]() {  // (uniform)
    if (ne > 0 && !row.bm) build_bitmap(row, hist + kBitmapOffset);
  };
  if (status == kPlanPoint) {
    const float xmax = val_of(mkey);
    // point rows: the first NaN, the first max (greedy), the first +inf z, or index 0 (all -inf)
    if (f.plan.nnan) {
      need_bitmap();
      k.point = find_first(row, [&](float x, int) -> u64 { return x != x; }, 0ull, srch);
    } else if (!(T > 0.0f)) {
      int pt = -1;
      if constexpr (SPLIT) {
        need_bitmap();
        pt = split_find(a, row, f, ne, xmax, 0ull, srch, hist + kMatchOffset, recs);
      } else if (!a.out_probs && cells_per(row) * kThreads <= 4 * kMatchWords) {  // (uniform)
        // the first id holding the max, by the member search from the kept low bytes (as the
        // draw's member) instead of a pass over the row
        uint8_t* cells = reinterpret_cast<uint8_t*>(hist + kMatchOffset);
        const int ncq = cells_per(row) * kThreads / 16;
        for (int i = tid; i < ncq; i += kThreads) reinterpret_cast<uint4*>(cells)[i] = make_uint4(0, 0, 0, 0);
        if (tid == 0) f.si[6] = -1;
        lds_barrier();
        pt = select_member(row, f, ne, xmax, 0ull, cells, mxk, low, sl, og, e0, estep);
      }
      if (pt < 0) {  // (uniform)
        need_bitmap();
        pt = find_first(row, [&](float x, int) -> u64 { return x == xmax; }, 0ull, srch);
      }
      k.point = pt;
    } else {
      need_bitmap();
      if (!degenerate(row, p, mkey, 0, mz, srch, k)) k.point = 0;
    }
    finish<STATE>(a, row, p, mz, k, 0, &srch.vslot, r);
    return true;
  }
  // ---- 5. [all] per-chunk masses of elements >= x0 ---------------------------------------
  {
    const float x0 = uniform_f(f.plan.x0);
    const uint32_t x0top = key_of(x0) >> 16;
    // wave w takes chunks w + 16 l (lane l says which need work) two at a time: lanes 0-31 the
    // first, lanes 32-63 the second, lane l the keys 2(l mod 32) and 2(l mod 32) + 1 of its chunk
    // (one histogram word holds both counts); fp64 exps for populated keys only
    const int wv = tid / kWave, l = lane_id();
    const int cl = wv + kWaves * l;
    const bool need = f.ccnt[cl] > 0 && 65535u - 64u * static_cast<uint32_t>(cl) >= x0top;
    u64 todo = __ballot(need);
    const bool second = l >= 32;
    const uint32_t l2 = static_cast<uint32_t>(l & 31);
    while (todo) {  // (uniform)
      const int i1 = __ffsll(static_cast<long long>(todo)) - 1;
      todo &= todo - 1;
      const int i2 = todo ? __ffsll(static_cast<long long>(todo)) - 1 : -1;
      todo &= todo - 1;
      const bool live = !second || i2 >= 0;
      const int c = wv + kWaves * (second && i2 >= 0 ? i2 : i1);
      // keys Ka (odd: the word's high half) and Ka - 1
      const uint32_t Ka = 65535u - 64u * static_cast<uint32_t>(c) - 2u * l2;
      const uint32_t hw = hist[Ka >> 1];
      const uint32_t na = live ? hw >> 16 : 0u, nb = live ? hw & 0xFFFFu : 0u;
      const float va = val16(Ka), vb = val16(Ka - 1u);
      // (no branch: both exps of a lane interleave; keys below x0 count 0)
      u64 mq = static_cast<u64>(va >= x0 ? na : 0u) * mass_q(ptilde(va, T, mz)) +
               static_cast<u64>(vb >= x0 ? nb : 0u) * mass_q(ptilde(vb, T, mz));
      mq = half_incl_scan<u64>(mq);
      if (l2 == 31u && live) atomicAdd(&f.cmass[c], mq);
    }
    for (int e = tid; e < ne; e += kThreads) {
      const float x = f.eval[e];
      if (x >= x0) atomicAdd(&f.cmass[chunk_of16(key_of(x) >> 16)], mass_q(ptilde(x, T, mz)));
    }
  }
  lds_barrier();
  // ---- 6/7. [wave 0] the total, the top-p cutoff, the draw ---------------------------------
  if (tid < kWave) {
    const int l = tid;
    int status2 = kPlanFast;
    float x0 = f.plan.x0;
    // lane l sums chunks 16l .. 16l + 15; a search inside the chunks of one lane L then gives
    // lane i of every 16-lane row chunk 16L + i and the mass above it
    u64 sum = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint4 v4 = *reinterpret_cast<const uint4*>(&f.cmass[16 * l + 2 * q]);
      sum += ((static_cast<u64>(v4.y) << 32) | v4.x) + ((static_cast<u64>(v4.w) << 32) | v4.z);
    }
    const u64 incl = wave_incl_scan<u64>(sum);
    const u64 S0 = dpp::last(incl);
    const u64 base = incl - sum;  // mass above chunk 16l
    auto lane_chunks = [&](int L, u64& mq, u64& run) {
      mq = f.cmass[16 * L + (l & 15)];
      run = readlane64(base, L) + row_incl_scan<u64>(mq) - mq;
    };
    Kept kk;
    kk.x0 = x0;
    kk.S = S0;
    if (p.tp < 1.0f) {
      const double P = static_cast<double>(p.tp) * static_cast<double>(S0);
      // the last chunk holding mass whose mass above is < P: the chunks with mass above < P are
      // a prefix, so it is in the last lane whose first chunk has mass above < P when that lane
      // holds mass (its first chunk holding mass has that lane's mass above), else it is the
      // last chunk holding mass of the lanes before
      int c = -1;
      u64 ab = 0;
      const u64 below = __ballot(static_cast<double>(base) < P);
      if (below) {
        const int lb = 63 - __clzll(static_cast<long long>(below));
        const bool in_lb = readlane64(sum, lb) > 0;
        const u64 held = __ballot(sum > 0 && l < lb);
        const int L = in_lb ? lb : (held ? 63 - __clzll(static_cast<long long>(held)) : -1);
        if (L >= 0) {
          u64 mq, run;
          lane_chunks(L, mq, run);
          const u64 hm = __ballot(mq > 0 && (!in_lb || static_cast<double>(run) < P)) & 0xFFFFull;
          const int q = 63 - __clzll(static_cast<long long>(hm));  // (hm != 0: the lane holds mass)
          c = 16 * L + q;
          ab = readlane64(run, q);
        }
      }
      if (c < 0) {
        status2 = kPlanGeneric;
      } else {
        const WalkResult wr = wave_walk(hist, f, ne, c, kWalkCutoff, ab, P, x0, T, mz);
        if (!wr.ok) {
          status2 = kPlanGeneric;
        } else {
          kk.has_cut = true;
          kk.vc = val_of(wr.key);
          kk.qc = wr.q;
          kk.mabove_c = wr.above;
          uint32_t rr = wr.n;
          if (kk.qc > 0) {
            const double cr = ceil((P - static_cast<double>(wr.above)) / static_cast<double>(kk.qc));
            rr = cr < 1.0 ? 1u : (cr >= static_cast<double>(wr.n) ? wr.n : static_cast<uint32_t>(cr));
          }
          kk.r = rr;
          kk.partial = rr < wr.n;
          if (!kk.partial) kk.x0 = kk.vc;
          kk.S = wr.above + static_cast<u64>(rr) * kk.qc;
        }
      }
    }
    // the draw's value group: descending value, ascending id within a value
    float vd = 0.0f;
    u64 j = 0;
    if (status2 == kPlanFast && !a.out_probs) {
      const float u = p.u >= 0.0f ? p.u : 0.0f;
      const u64 td0 = static_cast<u64>(static_cast<double>(u) * static_cast<double>(kk.S));
      const u64 td = td0 < kk.S ? td0 : kk.S - 1;
      if (kk.has_cut && td >= kk.mabove_c && kk.qc > 0) {
        vd = kk.vc;
        j = div_index(td - kk.mabove_c, kk.qc);
      } else {
        // the chunk holding the target (in the lane whose mass range holds it), then the value
        // inside it
        int cd = -1;
        u64 abd = 0;
        const u64 hl = __ballot(sum > 0 && base <= td && td < base + sum);
        if (hl) {
          const int L = __ffsll(static_cast<long long>(hl)) - 1;
          u64 mq, run;
          lane_chunks(L, mq, run);
          const u64 hm = __ballot(mq > 0 && run <= td && td < run + mq) & 0xFFFFull;
          if (hm) {
            const int q = __ffsll(static_cast<long long>(hm)) - 1;
            cd = 16 * L + q;
            abd = readlane64(run, q);
          }
        }
        if (cd < 0) {
          status2 = kPlanGeneric;
        } else {
          const WalkResult wr = wave_walk(hist, f, ne, cd, kWalkCross, abd, static_cast<double>(td), x0, T, mz);
          if (!wr.ok) {
            status2 = kPlanGeneric;
          } else {
            vd = val_of(wr.key);
            j = wr.q ? div_index(td - wr.above, wr.q) : 0ull;
            if (j >= wr.n) j = wr.n ? wr.n - 1 : 0;
          }
        }
      }
    }
    if (l == 0) {
      f.plan.status = status2;
      f.plan.x0 = kk.x0;
      f.plan.vc = kk.vc;
      f.plan.partial = kk.partial;
      f.plan.has_cut = kk.has_cut;
      f.plan.r = kk.r;
      f.plan.mabove_c = kk.mabove_c;
      f.plan.qc = kk.qc;
      f.plan.S = kk.S;
      f.plan.vd = vd;
      f.plan.j = j;
    }
  }
  lds_barrier();
  if (f.plan.status == kPlanGeneric) return false;
  k.x0 = f.plan.x0;
  k.vc = f.plan.vc;
  k.partial = f.plan.partial;
  k.has_cut = f.plan.has_cut;
  k.r = f.plan.r;
  k.mabove_c = f.plan.mabove_c;
  k.qc = f.plan.qc;
  k.S = f.plan.S;
  const float vd = f.plan.vd;
  const u64 j = f.plan.j;
  // One pass zeroes the member search's cells and, when a pass over the row will need it, the
  // position bitmap of the penalised ids.
  const bool cells_fit = !SPLIT && !a.out_probs && cells_per(row) * kThreads <= 4 * kMatchWords;
  const bool bitmap_now = ne > 0 && !cells_fit;  // (uniform)
  {
    uint32_t* bmw = hist + kBitmapOffset;
    // (16-byte stores: both regions start 16-byte aligned, and the bitmap's last quad stays in
    // its region)
    const int nbq = bitmap_now ? (row.nblk + 15) / 16 : 0;
    const int ncq = cells_fit ? cells_per(row) * kThreads / 16 : 0;
    for (int i = tid; i < nbq; i += kThreads) reinterpret_cast<uint4*>(bmw)[i] = make_uint4(0, 0, 0, 0);
    for (int i = tid; i < ncq; i += kThreads) reinterpret_cast<uint4*>(hist + kMatchOffset)[i] = make_uint4(0, 0, 0, 0);
    if (tid == 0) f.si[6] = -1;
    lds_barrier();
    if (bitmap_now) {
      for (int e = tid; e < ne; e += kThreads) {
        const uint32_t id = static_cast<uint32_t>(f.eid[e]);
        atomicOr(&bmw[id >> 5], 1u << (id & 31u));
      }
      lds_barrier();
      row.bm = reinterpret_cast<const uint8_t*>(bmw);
    }
  }
  // the partial cutoff group's r-th member (row states, probabilities, a draft inside that group):
  // the member search from the kept low bytes, as for the draw, where its cells fit (then cleared
  // again for the draw's search), else a pass over the row
  if (k.partial) {
    bool need = STATE || a.out_probs != nullptr;
    if (!need && p.draft >= 0 && p.draft < row.V && a.out_dprob) need = value_of(row, p.draft, &srch.vslot) == k.vc;
    if (need) {  // (uniform)
      int id = -1;
      if (cells_fit) {
        uint8_t* cells = reinterpret_cast<uint8_t*>(hist + kMatchOffset);
        id = select_member(row, f, ne, k.vc, static_cast<u64>(k.r - 1), cells, mxk, low, sl, og, e0, estep);
        lds_barrier();  // (every wave has read f.si[6] before thread 0 resets it for the draw's search)
        const int ncq = cells_per(row) * kThreads / 16;
        for (int i = tid; i < ncq; i += kThreads) reinterpret_cast<uint4*>(cells)[i] = make_uint4(0, 0, 0, 0);
        if (tid == 0) f.si[6] = -1;
        lds_barrier();
      }
      const float vc = k.vc;
      if (id < 0) {  // (uniform)
        need_bitmap();
        id = find_first(row, [&](float x, int) -> u64 { return x == vc; }, static_cast<u64>(k.r - 1), srch);
      }
      k.idr = id;
    }
  }
  int draw = 0;
  if (!a.out_probs) {
    if constexpr (SPLIT) draw = split_find(a, row, f, ne, vd, j, srch, hist + kMatchOffset, recs);
    else
      draw = cells_fit ? select_member(row, f, ne, vd, j, reinterpret_cast<uint8_t*>(hist + kMatchOffset), mxk, low,
                                       sl, og, e0, estep)
                       : -1;
    if (draw < 0) {  // (uniform)
      need_bitmap();
      draw = find_first(row, [&](float x, int) -> u64 { return x == vd; }, j, srch);
    }
  }
  finish<STATE>(a, row, p, mz, k, draw, &srch.vslot, r);
  return true;
}

// ---- rows decided from their tile maxima (vsamp_sample_tiles, vsamp_sample_tile_pass) ---------
// k_lm_head writes, beside the bf16 logits, the max of every kStatTile consecutive logits of a
// row (as a value: NaN the largest); the tile pass computes the same maxima of bf16 or fp32
// rows from any source. For some rows those maxima bound
// where every token the draw can keep lies, and the row is decided from a few tiles:
//   * greedy rows: the first id holding the row max lies in the first tile whose max equals the
//     row max (as values: -0 equals +0), and only that tile is read;
//   * rows sampled at T > 0 with top-k (K <= kSortCap) or min-p: every kept token has
//     x >= xlo, where for top-k xlo is the least x with fl(x / T) >= fl(theta / T), theta the
//     K-th largest tile max (the K largest tile maxima are K logits, so theta is at most the
//     K-th largest logit, whose z every kept token reaches), and for min-p the least x whose
//     p~ = exp(fl(x / T) - max z) reaches min_p; a kept token then lies in a tile whose max is
//     >= xlo. The elements >= xlo of those tiles (at most kTileRowTiles tiles, at most
//     kSortCap elements) are sorted as the generic path sorts its short lists, the exact top-k
//     and min-p thresholds taken from them, and sorted_tail finishes the row: the same
//     cutoff, masses and draw as a pass over the row.
// Rows with penalties, NaN maxima, infinite scaled logits, top-p alone, or more candidates than
// that take the row passes (the caller's path) as if no tile maxima were given.
constexpr int kStatTile = 128;      // logits per statistics tile (k_lm_head's column tile)
constexpr int kTileRowTiles = 64;   // candidate tiles a row decided from its tiles reads at most

// The key of the k-th largest (1-based, with multiplicity) of the 16-bit keys keys[0 .. nk) of
// every thread (nk <= 4; k <= the number of keys): two rounds over the high and the low byte,
// each a 256-bin LDS histogram (h0, then h1: both zeroed at the start) that wave 0 walks from
// the top. `h0` and `h1` are 256 words each, `sh` 4 words.
__device__ __forceinline__ uint32_t kth_key16(const uint32_t (&keys)[4], int nk, uint32_t k, uint32_t* h0, uint32_t* h1,
                                              uint32_t* sh) {
  const int tid = threadIdx.x;
  uint32_t hi = 0, above = 0;
  if (tid < 256) h0[tid] = 0;
  else if (tid < 512) h1[tid - 256] = 0;
  lds_barrier();
  for (int round = 0; round < 2; ++round) {
    uint32_t* h = round == 0 ? h0 : h1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i < nk && (round == 0 || (keys[i] >> 8) == hi)) atomicAdd(&h[round == 0 ? keys[i] >> 8 : keys[i] & 0xFFu], 1u);
    }
    lds_barrier();
    if (tid < kWave) {
      // lane l: bins 255 - 4l .. 252 - 4l, descending
      uint32_t c[4], s4 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = h[255 - 4 * tid - i];
        s4 += c[i];
      }
      uint32_t ex = above + wave_incl_scan<uint32_t>(s4) - s4;
      if (ex < k && k <= ex + s4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (ex < k && k <= ex + c[i]) {
            sh[0] = static_cast<uint32_t>(255 - 4 * tid - i);
            sh[1] = ex;
          }
          ex += c[i];
        }
      }
    }
    lds_barrier();
    if (round == 0) hi = sh[0];
    above = sh[1];
  }
  return (hi << 8) | sh[0];
}

// The tile maxima of bf16 or fp32 rows from any source (what k_lm_head's epilogue writes beside its
// logits): the max of every kStatTile consecutive logits of a row, as a value (ordered keys: a
// NaN is the largest; -0.0 and +0.0 are one value). Sixteen lanes take a tile, eight logits a
// lane, and reduce over their 16-lane row; grid (ceil(nT / 16), B) of 256-thread workgroups, so
// even one row spreads over the chip.
constexpr int kTileFusedWorkgroups = 256;  // (one round on the CUs; vsamp_sample_tile_pass)
constexpr int kTileMaxThreads = 256;
constexpr int kTilesPerBlock = kTileMaxThreads / 16;
// A lane's eight logits of a tile (16-byte loads: one of bf16, two of fp32) and their largest key:
// the key of their IEEE maximum (-0 below +0, as in key order), or, when a NaN among them makes
// that maximum a NaN, the largest of their keys.
template <class Tin>
constexpr int kTileLoads = sizeof(Tin) == 2 ? 1 : 2;
template <class Tin>
__device__ __forceinline__ uint32_t lane_tile_key(const uint4 (&v)[kTileLoads<Tin>]) {
  float x[kBlk];
#pragma unroll
  for (int j = 0; j < kTileLoads<Tin>; ++j) {
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (sizeof(Tin) == 2) {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      } else {
        x[4 * j + i] = __uint_as_float(w[i]);
      }
    }
  }
  const float bx = max_of8(x);
  uint32_t mk = key_of(bx);
  if (bx != bx) {
    mk = 0;  // (below every key)
#pragma unroll
    for (int i = 0; i < kBlk; ++i) mk = max(mk, key_of(x[i]));
  }
  return mk;
}
// The same for a lane whose eight logits are not one aligned run inside the row: element by
// element (fewer past the end).
template <class Tin>
__device__ __forceinline__ uint32_t lane_tile_key_each(const Tin* row, int i0, int V) {
  uint32_t mk = 0;
  for (int i = i0; i < i0 + 8 && i < V; ++i) mk = max(mk, key_of(load_one<Tin>(row, i)));
  return mk;
}

template <class Tin>
__global__ __launch_bounds__(kTileMaxThreads) void k_tile_max(const Tin* logits, int64_t stride, int V, int nT,
                                                             float* out) {
  const int r = blockIdx.y;
  const int l16 = threadIdx.x & 15;
  const int t = blockIdx.x * kTilesPerBlock + (threadIdx.x >> 4);  // (the same in a 16-lane row)
  const Tin* row = as_global(logits) + static_cast<int64_t>(r) * stride;
  const int i0 = t * kStatTile + 8 * l16;  // this lane's first logit
  uint32_t mk = 0;                         // (below every key)
  if (t < nT) {
    if ((reinterpret_cast<uintptr_t>(row + i0) & 15u) == 0 && i0 + 8 <= V) {
      uint4 q[kTileLoads<Tin>];
#pragma unroll
      for (int j = 0; j < kTileLoads<Tin>; ++j) q[j] = ld_global_u4(reinterpret_cast<const uint4*>(row + i0) + j);
      mk = lane_tile_key<Tin>(q);
    } else {
      mk = lane_tile_key_each<Tin>(row, i0, V);
    }
  }
  auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  mk = umax(mk, dpp::mov<dpp::kXor1>(mk));
  mk = umax(mk, dpp::mov<dpp::kXor2>(mk));
  mk = umax(mk, dpp::mov<dpp::kHalfMirror>(mk));
  mk = umax(mk, dpp::mov<dpp::kMirror>(mk));
  if (t < nT && l16 == 0) as_global(out)[static_cast<int64_t>(r) * nT + t] = val_of(mk);
}

// (the fused tile pass) Workgroup g of row r's G computes the maxima of tiles g * per .. (per =
// ceil(nT / G), at most kTileSharePasses * 64: sixteen lanes a tile as k_tile_max, up to
// kTileSharePasses runs of eight logits per thread, their 16-byte loads (one a run of bf16, two
// of fp32) issued before any is used) into a.tile_max with
// device-coherent stores; waits for them; then thread 0 counts the workgroup in at the row's
// arrival word. The last of the G resets the word to 0 (nothing else touches it in this launch)
// and returns true: it finishes the row, the others return false and exit. `flag` is an LDS word.
// One pass (at most 64 tiles a workgroup): more workgroups a row measured faster than four passes
// (a CU reading 16 KB of the row instead of 64 KB; 11.7 against 13.2 us for one 151936-logit row).
constexpr int kTileSharePasses = 1;
template <class Tin>
__device__ __forceinline__ bool tile_share(const SampleArgs& a, int r, int g, int* flag) {
  const int G = a.tile_G, nT = a.nT;
  const int per = (nT + G - 1) / G;
  const int end = min(nT, (g + 1) * per);
  const int l16 = threadIdx.x & 15;
  const Tin* row = as_global(static_cast<const Tin*>(a.logits)) + static_cast<int64_t>(r) * a.stride;
  const int V = a.V;
  float* out = const_cast<float*>(a.tile_max) + static_cast<int64_t>(r) * nT;
  // pass q: tile g * per + threadIdx.x / 16 + 64 q (the same in a 16-lane row); whole aligned
  // 16-byte chunks are loaded first (every lane issues its loads: one that has none reads a
  // constant aligned block, unused), the rest element by element
  uint4 v[kTileSharePasses][kTileLoads<Tin>];
  bool whole[kTileSharePasses];
#pragma unroll
  for (int q = 0; q < kTileSharePasses; ++q) {
    const int t = g * per + static_cast<int>(threadIdx.x >> 4) + kWave * q;
    const int i0 = t * kStatTile + 8 * l16;
    whole[q] = t < end && (reinterpret_cast<uintptr_t>(row + i0) & 15u) == 0 && i0 + 8 <= V;
#pragma unroll
    for (int j = 0; j < kTileLoads<Tin>; ++j)
      v[q][j] = ld_global_u4(whole[q] ? reinterpret_cast<const uint4*>(row + i0) + j
                                      : reinterpret_cast<const uint4*>(g_unused_block));
  }
  auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
#pragma unroll
  for (int q = 0; q < kTileSharePasses; ++q) {
    const int t = g * per + static_cast<int>(threadIdx.x >> 4) + kWave * q;
    uint32_t mk = 0;  // (below every key)
    if (whole[q]) mk = lane_tile_key<Tin>(v[q]);
    else if (t < end) mk = lane_tile_key_each<Tin>(row, t * kStatTile + 8 * l16, V);
    mk = umax(mk, dpp::mov<dpp::kXor1>(mk));
    mk = umax(mk, dpp::mov<dpp::kXor2>(mk));
    mk = umax(mk, dpp::mov<dpp::kHalfMirror>(mk));
    mk = umax(mk, dpp::mov<dpp::kMirror>(mk));
    if (t < end && l16 == 0) st_dev<float>(out + t, val_of(mk));
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();  // (every thread's stores have completed)
  if (threadIdx.x == 0) {
    uint32_t* word = a.tile_arrive + r;
    const uint32_t old = __hip_atomic_fetch_add(word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == static_cast<uint32_t>(G - 1);
    if (last) st_dev<uint32_t>(word, 0u);
    *flag = last ? 1 : 0;
  }
  __syncthreads();
  return *flag != 0;
}

// Whether a fused tile pass computes a row's maxima: greedy rows and top-k rows (0 < K <= kSortCap,
// K < V) without penalties, whose candidates the maxima bound; rows with top-p or min-p alone keep
// a share of the row that depends on its values (hundreds to thousands of tokens) and go to the
// row passes directly.
template <bool PEN>
__device__ __forceinline__ bool tile_candidate(const SampleArgs& a, const RowParams& p) {
  const bool pen_on = PEN && p.h1 > p.h0 && (p.rep != 1.0f || p.pres != 0.0f || p.freq != 0.0f);
  if (pen_on || a.out_probs || a.out_state || a.nT > 4 * kThreads) return false;
  if (!(p.T > 0.0f)) return true;
  return p.K > 0 && p.K < a.V && p.K <= kSortCap && p.K <= a.nT;
}

// Returns true when the row was decided (outputs written) from its tile maxima; false, having
// written nothing, when it needs the row passes. Every thread calls; `p.u` is clamped to >= 0.
template <bool PEN, class Tin>
__device__ __forceinline__ bool tile_row(const SampleArgs& a, const Row<Tin>& row, const RowParams& p, GenericSmem& g,
                                         int r) {
  const int tid = threadIdx.x;
  const int V = row.V;
  const int nT = a.nT;
  const bool pen_on = PEN && p.h1 > p.h0 && (p.rep != 1.0f || p.pres != 0.0f || p.freq != 0.0f);
  const bool greedy = !(p.T > 0.0f);
  const bool topk = p.K > 0 && p.K < V;
  // (uniform)
  if (pen_on || a.out_probs || a.out_state || nT > 4 * kThreads) return false;
  if (!greedy && (!(topk || p.mp > 0.0f) || (topk && (p.K > kSortCap || p.K > nT)))) return false;
  uint32_t* sh = g.rdx.bk;
  // the tile maxima: thread t takes tiles t + i * kThreads
  const float* tm = a.tile_max + static_cast<int64_t>(r) * nT;
  float mt[4];
  uint32_t kt[4];
  uint32_t mk = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = tid + i * kThreads;
    mt[i] = t < nT ? ld_dev(tm + t) : -INFINITY;  // (device-coherent: other workgroups of a fused pass wrote them)
  }
  Kept k;
  if (greedy) {
    // the row max and the first tile holding it in one reduction (key above the complemented
    // tile: equal values, -0 and +0 included, have one key), then that tile's first element equal
    // to it, by wave 0 (two elements a lane)
    u64 best = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = tid + i * kThreads;
      const u64 v = t < nT ? (static_cast<u64>(key_of(mt[i])) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(t)) : 0ull;
      best = v > best ? v : best;
    }
    best = block_max_u64(best, g.srch.red64);
    mk = static_cast<uint32_t>(best >> 32);
    if (mk > key_of(INFINITY)) return false;  // a NaN: the row passes find the first one
    const float M = val_of(mk);
    const uint32_t first = 0xFFFFFFFFu - static_cast<uint32_t>(best);
    if (tid < kWave) {
      uint32_t id = 0xFFFFFFFFu;
#pragma unroll
      for (int h = 1; h >= 0; --h) {
        const int i = static_cast<int>(first) * kStatTile + tid + h * kWave;
        if (i < V && load_one<Tin>(row.p, i) == M) id = static_cast<uint32_t>(i);
      }
      id = dpp::reduce(id, [](uint32_t x, uint32_t y) { return x < y ? x : y; });
      if (tid == 0) sh[0] = id;
    }
    lds_barrier();
    const uint32_t id = sh[0];
    if (id >= static_cast<uint32_t>(V)) return false;  // (tile maxima not of these logits)
    k.point = static_cast<int>(id);
    finish<false>(a, row, p, 0.0f, k, 0, &g.srch.vslot, r);
    return true;
  }
  // Top-k rows count their tiles' maxima by the top 12 bits of their keys (4096 bins in LDS; of
  // a bf16 value, the top 12 bits of its 16-bit key): the lowest value of the bin holding the
  // K-th largest is at most the K-th largest tile max, so at most the K-th largest logit. The row
  // max rides the same barrier (one LDS atomicMax per wave).
  uint32_t* h12 = reinterpret_cast<uint32_t*>(&g) + kBitmapOffset;
  uint32_t* smax = &g.rdx.ncand;
  uint32_t* tcount = reinterpret_cast<uint32_t*>(g.rdx.bq);  // (the candidate tiles' count)
  if (topk) reinterpret_cast<uint4*>(h12)[tid] = make_uint4(0, 0, 0, 0);
  if (tid == 0) *smax = 0;
  lds_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = tid + i * kThreads;
    kt[i] = t < nT ? key_of(mt[i]) : 0u;  // (0: below every key)
    mk = kt[i] > mk ? kt[i] : mk;
    if (topk && t < nT) atomicAdd(&h12[kt[i] >> 20], 1u);
  }
  mk = dpp::reduce(mk, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
  if (lane_id() == 0) atomicMax(smax, mk);
  lds_barrier();
  mk = *smax;
  if (mk > key_of(INFINITY)) return false;  // a NaN: the row passes find the first one
  const float M = val_of(mk);
  const float T = p.T;
  const float mz = M / T;
  if (!(mz > -INFINITY && mz < INFINITY)) return false;  // point rows: the row passes
  // xlo: no kept token lies below it (wave 0 decides; the others wait at the barrier)
  const uint32_t lo_key = key_of(-INFINITY);
  if (tid < kWave) {
    float xlo = -INFINITY, xm = -INFINITY;
    if (topk) {
      // the bin of the K-th largest: lane l sums bins 4095 - 64 l - 63 .. 4095 - 64 l (lane 0
      // the top ones), then lane i of the crossing lane's 64 bins takes bin 4095 - 64 L - i
      const uint32_t K = static_cast<uint32_t>(p.K);
      const int l = tid;
      uint32_t sum = 0;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const uint4 v = reinterpret_cast<const uint4*>(h12 + 4032 - 64 * l)[q];
        sum += v.x + v.y + v.z + v.w;
      }
      const uint32_t incl = wave_incl_scan<uint32_t>(sum);
      const int L = __ffsll(static_cast<long long>(__ballot(incl >= K))) - 1;  // (K <= nT: some lane crosses)
      const uint32_t above = __builtin_amdgcn_readlane(incl, L) - __builtin_amdgcn_readlane(sum, L);
      const uint32_t c = h12[4095 - 64 * L - l];
      const uint32_t incl2 = above + wave_incl_scan<uint32_t>(c);
      const int i = __ffsll(static_cast<long long>(__ballot(incl2 >= K))) - 1;
      const uint32_t bin = static_cast<uint32_t>(4095 - 64 * L - i);
      // the least value of the bin (not below -inf): of bf16 rows, the bf16 value of its least
      // 16-bit key; of fp32 rows, the value of its least 32-bit key
      float theta;
      if constexpr (sizeof(Tin) == 2) {
        const uint32_t k16 = (bin << 4) > 0x007Fu ? (bin << 4) : 0x007Fu;
        theta = val16(k16);
      } else {
        const uint32_t k32 = (bin << 20) > key_of(-INFINITY) ? (bin << 20) : key_of(-INFINITY);
        theta = val_of(k32);
      }
      const float zt = theta / T;
      xlo = val_of(wave_bisect(lo_key, key_of(theta), key_of(zt * T), [&](float x) { return x / T >= zt; }));
    }
    if (p.mp > 0.0f) {
      const double dmp = static_cast<double>(p.mp);
      const float guess = T * (mz + __logf(p.mp));
      xm = val_of(wave_bisect(lo_key, mk, key_of(guess), [&](float x) { return ptilde(x, T, mz) >= dmp; }));
    }
    if (tid == 0) {
      reinterpret_cast<float*>(sh)[0] = xlo > xm ? xlo : xm;
      reinterpret_cast<float*>(sh)[1] = xm;
      *tcount = 0;
    }
  }
  lds_barrier();
  const float xlo = reinterpret_cast<const float*>(sh)[0];
  const float xm = reinterpret_cast<const float*>(sh)[1];
  // the tiles that can hold a kept token, listed in LDS in any order (one counter update per
  // wave and ballot)
  int* ctile = reinterpret_cast<int*>(g.srch.tw);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = tid + i * kThreads;
    const bool in = t < nT && mt[i] >= xlo;
    const u64 bal = __ballot(in);
    if (bal) {  // (uniform over the wave)
      const int leader = __ffsll(static_cast<long long>(bal)) - 1;
      uint32_t pos = 0;
      if (lane_id() == leader) pos = atomicAdd(tcount, static_cast<uint32_t>(__popcll(bal)));
      pos = __builtin_amdgcn_readlane(pos, leader) + static_cast<uint32_t>(__popcll(bal & ((1ull << lane_id()) - 1ull)));
      if (in && pos < static_cast<uint32_t>(kTileRowTiles)) ctile[pos] = t;
    }
  }
  if (tid == 0) sh[2] = 0;
  lds_barrier();
  const uint32_t ntile = *tcount;
  if (ntile > static_cast<uint32_t>(kTileRowTiles)) return false;  // (uniform)
  // their elements >= xlo, into the candidate list (every element's load first)
  Cand* c = reinterpret_cast<Cand*>(reinterpret_cast<uint32_t*>(&g) + kMatchOffset);
  constexpr int kPer = kTileRowTiles * kStatTile / kThreads;
  float xs[kPer];
  int ids[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int e = tid + q * kThreads;
    ids[q] = e < static_cast<int>(ntile) * kStatTile ? ctile[e / kStatTile] * kStatTile + e % kStatTile : V;
    xs[q] = load_one<Tin>(row.p, ids[q] < V ? ids[q] : 0);
  }
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const bool in = ids[q] < V && xs[q] >= xlo;
    const u64 bal = __ballot(in);  // (one counter update per wave)
    if (bal) {
      const int leader = __ffsll(static_cast<long long>(bal)) - 1;
      uint32_t pos = 0;
      if (lane_id() == leader) pos = atomicAdd(&sh[2], static_cast<uint32_t>(__popcll(bal)));
      pos = __builtin_amdgcn_readlane(pos, leader) + static_cast<uint32_t>(__popcll(bal & ((1ull << lane_id()) - 1ull)));
      if (in && pos < static_cast<uint32_t>(kSortCap)) c[pos] = Cand{xs[q], ids[q]};
    }
  }
  lds_barrier();
  const int n = static_cast<int>(sh[2]);
  if (n > kSortCap || n < 1) return false;  // (uniform)
  sort_cands(c, n, c + kCandCap);
  // the exact thresholds: the K-th largest element's z (when the list holds K elements; else
  // min-p's threshold, above the K-th largest, binds) and min-p's
  if (tid < kWave) {
    float x0 = xm;
    if (topk && n >= p.K) {
      const float kz = c[p.K - 1].x / T;
      const float xk = val_of(wave_bisect(lo_key, key_of(c[p.K - 1].x), key_of(kz * T), [&](float x) { return x / T >= kz; }));
      x0 = xk > x0 ? xk : x0;
    }
    if (tid == 0) reinterpret_cast<float*>(sh)[3] = x0;
  }
  lds_barrier();
  k.x0 = reinterpret_cast<const float*>(sh)[3];
  return sorted_tail<false>(a, row, p, g, g.srch, c, n, mz, k, r);
}

__device__ __forceinline__ SampleArgs globalized(SampleArgs a) {
  a.logits = as_global(a.logits);
  a.temp = as_global(a.temp);
  a.topk = as_global(a.topk);
  a.topp = as_global(a.topp);
  a.minp = as_global(a.minp);
  a.u = as_global(a.u);
  a.draft = as_global(a.draft);
  a.out_ids = as_global(a.out_ids);
  a.hist_out = as_global(a.hist_out);
  a.out_dprob = as_global(a.out_dprob);
  a.out_probs = as_global(a.out_probs);
  a.out_state = as_global(a.out_state);
  a.ws = globalized(a.ws);
  a.off = as_global(a.off);
  a.pen = globalized(a.pen);
  a.slices = as_global(a.slices);
  a.arrive = as_global(a.arrive);
  a.tile_max = as_global(a.tile_max);
  a.tile_arrive = as_global(a.tile_arrive);
  return a;
}

// STATE: also write each row's RowState (the speculative verify's launches; never with PEN).
// SPLIT: a bf16 split-row launch (grid B * G).
// TILES: rows (bf16 or fp32) with their tile maxima (a.tile_max): the rows tile_row can decide
// are decided from a few tiles, the others take the row passes below.
template <class Tin, bool PEN, bool STATE = false, bool SPLIT = false, bool TILES = false>
__global__ __launch_bounds__(kThreads) void k_sample(SampleArgs a_) {
  const SampleArgs a = globalized(a_);
  // 128 KB: the key histogram (or the generic path's penalty counts), then the id-search /
  // radix scratch
  __shared__ __align__(16) uint32_t big[kChunk];
  __shared__ FastSmem f;
  static_assert(sizeof(GenericSmem) <= sizeof(uint32_t) * kBitmapOffset, "scratch must fit below the bitmap");
  static_assert(kMatchOffset + kMatchWords <= kChunk, "count cells must fit");
  const bool fused = TILES && a.tile_arrive != nullptr;  // (uniform)
  const int r = SPLIT ? row_index(a) : fused ? static_cast<int>(blockIdx.x) / a.tile_G : static_cast<int>(blockIdx.x);
  const int tid = threadIdx.x;
  exp_table_init();  // (published by the first barrier of either path)
  // the row's parameters: thread w < kParamWords loads word w, the others word 0 (every thread
  // loads: a load on one branch only would make later waits wait for every load in flight)
  const uint32_t pw = param_word<PEN, STATE>(a, r, tid < kParamWords ? tid : 0);
  __builtin_amdgcn_sched_barrier(0);  // (issued before the row's first loads)

  Row<Tin> row;
  row.p = static_cast<const Tin*>(a.logits) + static_cast<int64_t>(r) * a.stride;
  row.V = a.V;
  row.nblk = (a.V + kBlk - 1) / kBlk;
  row.nstripes = (row.nblk + kThreads - 1) / kThreads;
  row.vec = (reinterpret_cast<uintptr_t>(row.p) & 15u) == 0;
  row.nexc = 0;
  row.bm = nullptr;  // built in LDS by the path that masks penalised positions
  row.eid = f.eid;   // the fast path keeps the penalised ids and values in LDS
  row.eval = f.eval;
  GenericSmem& g = *reinterpret_cast<GenericSmem*>(big);
  if constexpr (TILES && !STATE && !SPLIT) {
    if (tid < kParamWords) reinterpret_cast<uint32_t*>(&f.prm)[tid] = pw;
    lds_barrier();
    RowParams pt = f.prm;
    pt.u = pt.u >= 0.0f ? pt.u : 0.0f;
    // (a fused pass) a row the maxima can decide: this workgroup's share of its tile maxima, and
    // the row's last workgroup goes on; another row: its first workgroup runs the row passes and
    // the others exit
    bool try_tiles = true;
    if (fused) {
      const int gi = static_cast<int>(blockIdx.x) % a.tile_G;
      try_tiles = tile_candidate<PEN>(a, pt);  // (uniform)
      if (try_tiles ? !tile_share<Tin>(a, r, gi, &f.si[7]) : gi != 0) return;
    }
    if (try_tiles) {
      if (tile_row<PEN, Tin>(a, row, pt, g, r)) return;
      lds_barrier();  // (every thread is done with the tile path's LDS)
    }
  }
  if constexpr (sizeof(Tin) == 2) {
    if (fast_row<PEN, STATE, SPLIT>(a, row, f.prm, big, f, g.srch, pw, r)) return;
    lds_barrier();  // (every thread is done with the fast path's LDS; f.prm is set)
  } else {
    if (tid < kParamWords) reinterpret_cast<uint32_t*>(&f.prm)[tid] = pw;
    lds_barrier();
  }
  RowParams p = f.prm;
  p.u = p.u >= 0.0f ? p.u : 0.0f;
  // the generic path: the penalty pass writes the penalised ids and values to the workspace
  int ne = 0;
  bool have_bitmap = false;
  if (PEN) ne = static_cast<int>(penalty_phase<Tin>(a.pen, r, big, f.red32, ExcCache{nullptr, nullptr, 0}, &have_bitmap));
  __syncthreads();
  if (ne > 0) {
    row.nexc = ne;
    row.eid = a.ws.exc_id + p.h0;
    row.eval = a.ws.exc_val + p.h0;
  }
  generic_row<STATE>(a, row, p, g, f, r, have_bitmap);
}

}  // namespace vs
