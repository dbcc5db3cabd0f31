// Penalty pass: each row's token history -> exact per-id counts -> penalised logits.
//
// The penalties are not in the engine (server/protocol.py:133-135 rejects them); their
// arithmetic follows vLLM's order, one fp32 rounding per step and no fused multiply-add:
//   x = x > 0 ? x / rep : x * rep;   x = x - freq * c;   x = x - pres       (for every c > 0)
//
// Workspace output for row r (ids with c > 0 are the row's "exceptions"), in no particular order:
//   n_exc[r]                         number of distinct history ids in [0, V)
//   exc_id/exc_val[h0 + e]           e-th exception (h0 = hist_offsets[r]; a row has at most L_r
//                                    of them, so the slots never overlap); exc_cnt[h0 + e] its
//                                    count where a counting path gathers from the workspace
#pragma once

#include "common.cuh"

namespace vs {

constexpr int kChunk = 32768;  // ids counted per LDS pass (128 KB of u32 counters)

struct Workspace {
  uint32_t* n_exc;   // [B]
  int32_t* exc_id;   // [H]
  float* exc_val;    // [H]
  int32_t* exc_cnt;  // [H] (the counting passes' own pairs for their gather; not always written)
};

struct PenaltyArgs {
  const void* logits;
  int64_t stride;
  int V;
  const float* rep;
  const float* pres;
  const float* freq;
  const int32_t* hist;
  const int32_t* off;
  int hstep;  // entries of `off` per row: 1 (CSR) or 2 (a [start, end) pair per row)
  Workspace ws;
  int32_t* dense_counts;  // optional [B][counts_stride]
  int64_t counts_stride;
};

// The same arguments with every pointer cast to the global address space.
__device__ __forceinline__ Workspace globalized(Workspace w) {
  w.n_exc = as_global(w.n_exc);
  w.exc_id = as_global(w.exc_id);
  w.exc_val = as_global(w.exc_val);
  w.exc_cnt = as_global(w.exc_cnt);
  return w;
}

__device__ __forceinline__ PenaltyArgs globalized(PenaltyArgs a) {
  a.logits = as_global(a.logits);
  a.rep = as_global(a.rep);
  a.pres = as_global(a.pres);
  a.freq = as_global(a.freq);
  a.hist = as_global(a.hist);
  a.off = as_global(a.off);
  a.ws = globalized(a.ws);
  a.dense_counts = as_global(a.dense_counts);
  return a;
}

// f(src[i], i) for every i in [0, n) of this thread (i = tid + j * kThreads), eight loads in
// flight at a time: a loop that uses each load as it is issued waits a memory round trip per
// iteration (16 of them for a history of 16K ids). Every load is issued, clamped into [0, n).
// GLOBAL: src is global memory (global loads); otherwise it may be LDS too (flat loads).
template <bool GLOBAL = true, class F>
__device__ __forceinline__ void for_each_id(const int32_t* src, int n, F f) {
  constexpr int kU = 8;
  for (int i0 = threadIdx.x; i0 < n; i0 += kU * kThreads) {
    int v[kU];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
      const int32_t* q = src + min(i0 + k * kThreads, n - 1);
      if constexpr (GLOBAL) v[k] = ld_global(q);
      else v[k] = *q;
    }
#pragma unroll
    for (int k = 0; k < kU; ++k)
      if (i0 + k * kThreads < n) f(v[k], i0 + k * kThreads);
  }
}

__device__ __forceinline__ float apply_penalty(float x, int c, float rep, float pres, float freq) {
  // Compiled with -ffp-contract=off: every operation below rounds on its own.
  x = (x > 0.0f) ? x / rep : x * rep;
  const float fc = freq * static_cast<float>(c);
  x = x - fc;
  x = x - pres;
  return x;
}

template <class Tin>
__device__ __forceinline__ float load_one(const Tin* p, int64_t i);
template <>
__device__ __forceinline__ float load_one<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_to_f32(p[i]);
}
template <>
__device__ __forceinline__ float load_one<float>(const float* p, int64_t i) {
  return p[i];
}

// Where the penalty pass leaves the row's penalised ids and values in LDS, for a caller that
// keeps them there (cap = 0: none). Rows with more than cap penalised ids are
// still complete in the workspace.
struct ExcCache {
  int32_t* id;
  float* val;
  int cap;
};

// Counting: through a presence bitmap of the vocabulary (bitmap_count, below) when the
// vocabulary, the history and its distinct ids fit; otherwise a history of at most kHashMaxL ids
// in an LDS hash table (16384 slots of (id, count), at most 75 % full), a longer one in windows
// of ids.
constexpr int kHashSlots = 16384;
constexpr int kHashMaxL = 12288;
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
// windowed counting: LDS words [0, 16384) counters (32768 ids as u16 pairs, or 16384 as u32),
// [16384, 17408) presence bits, then cached history ids and staged (id, count) pairs
constexpr int kCountWords = 16384;
constexpr int kHistCache = kChunk - kCountWords - 1024;

// The penalised values of exceptions [0, n), whose (id, count) pairs pair(e) gives (from LDS or
// the workspace): all loads of a thread are issued before any value is computed.
template <class Tin, class P>
__device__ __forceinline__ void gather_values(const PenaltyArgs& a, const Tin* row, int h0, uint32_t n, P pair,
                                              float rep, float pres, float freq, const ExcCache& ec) {
  constexpr int kU = 8;
  for (uint32_t e0 = threadIdx.x; e0 < n; e0 += kU * kThreads) {
    int id[kU], c[kU];
    float x[kU];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
      const uint32_t e = e0 + k * kThreads;
      const int2 q = e < n ? pair(e) : make_int2(0, 0);
      id[k] = q.x;
      c[k] = q.y;
    }
#pragma unroll
    for (int k = 0; k < kU; ++k) x[k] = e0 + k * kThreads < n ? load_one<Tin>(row, id[k]) : 0.0f;
#pragma unroll
    for (int k = 0; k < kU; ++k) {
      const uint32_t e = e0 + k * kThreads;
      if (e >= n) continue;
      const float xv = apply_penalty(x[k], c[k], rep, pres, freq);
      a.ws.exc_val[h0 + e] = xv;
      if (static_cast<int>(e) < ec.cap) {
        ec.id[e] = id[k];
        ec.val[e] = xv;
      }
    }
  }
}

// Histories of at most 65535 ids over a vocabulary of at most kBmMaxV ids: a presence bitmap of
// the vocabulary (one non-returning atomic per history id), the exclusive prefix of its 64-bit
// words' popcounts, then u16 counts indexed by the rank of an id among the distinct ids (prefix +
// popcount below it; a second pass over the history). Thread t owns bitmap words kBmPer * t ..
// + kBmPer - 1 and stages their ids in rank order in LDS, from where the workgroup writes the
// (id, count) pairs coalesced (each thread straight to the workspace when they do not fit).
// Returns false (having written nothing) when the distinct ids do not fit: the caller then counts
// another way. The arrays start at LDS word kPenBitmapOffset, so the bitmap (bit id of 32-bit word
// id / 32) is where the sampling kernel's generic path keeps its bitmap of penalised ids, and
// stays there on return.
constexpr int kBmPer = 4;                       // 64-bit bitmap words per thread
constexpr int kBmMaxV = 64 * kBmPer * kThreads;  // 262144
constexpr int kPenBitmapOffset = 5120;
template <class Tin>
__device__ __forceinline__ bool bitmap_count(const PenaltyArgs& a, uint32_t* lds, uint32_t* red, ExcCache ec, int h0,
                                             int L, int V, bool on, int32_t* dc, float rep, float pres, float freq,
                                             const Tin* row, const int32_t* hist, uint32_t* n_out) {
  const int tid = threadIdx.x;
  const int nw = (V + 63) / 64;  // 64-bit bitmap words
  uint32_t* words = lds + kPenBitmapOffset;
  constexpr int kRoom = kChunk - kPenBitmapOffset;  // words from the bitmap on
  u64* bm = reinterpret_cast<u64*>(words);
  const int head = 2 * nw + (nw + 1) / 2;
  uint16_t* pre = reinterpret_cast<uint16_t*>(words + 2 * nw);  // u16 prefix per word
  uint32_t* cnt = words + head;                                  // u16 counts by rank, in pairs
  const int cap = 2 * (kRoom - head);                            // ranks that fit
  for (int i = tid; i < 2 * nw; i += kThreads) words[i] = 0;
  lds_barrier();
  for_each_id(hist, L, [&](int id, int) {
    if (id >= 0 && id < V) atomicOr(&words[id >> 5], 1u << (id & 31));
  });
  lds_barrier();
  u64 w[kBmPer];
  uint32_t n = 0;
#pragma unroll
  for (int k = 0; k < kBmPer; ++k) {
    const int wi = kBmPer * tid + k;
    w[k] = wi < nw ? bm[wi] : 0ull;
    n += __popcll(w[k]);
  }
  uint32_t total;
  const uint32_t e0 = block_excl_scan<uint32_t>(n, red, &total);
  if (total > static_cast<uint32_t>(cap) || total > 0xFFFFu) return false;  // (uniform)
  uint32_t pw[kBmPer];
  {
    uint32_t e = e0;
#pragma unroll
    for (int k = 0; k < kBmPer; ++k) {
      pw[k] = e;
      const int wi = kBmPer * tid + k;
      if (wi < nw) pre[wi] = static_cast<uint16_t>(e);
      e += __popcll(w[k]);
    }
  }
  for (int i = tid; i < static_cast<int>((total + 1) / 2); i += kThreads) cnt[i] = 0;
  lds_barrier();
  for_each_id(hist, L, [&](int id, int) {
    if (id < 0 || id >= V) return;
    const int wi = id >> 6;
    const uint32_t rank = pre[wi] + static_cast<uint32_t>(__popcll(bm[wi] & ((1ull << (id & 63)) - 1ull)));
    atomicAdd(&cnt[rank >> 1], 1u << ((rank & 1u) << 4));
  });
  lds_barrier();
  auto count_of = [&](uint32_t e) -> int { return static_cast<int>((cnt[e >> 1] >> ((e & 1u) << 4)) & 0xFFFFu); };
  // (id, count) pairs in rank order
  int32_t* rid = reinterpret_cast<int32_t*>(cnt + (total + 1) / 2);
  const uint32_t room = static_cast<uint32_t>(kRoom - head - static_cast<int>((total + 1) / 2));
  if (total <= room) {  // (uniform)
#pragma unroll
    for (int k = 0; k < kBmPer; ++k) {
      uint32_t e = pw[k];
      for (u64 m = w[k]; m; m &= m - 1) rid[e++] = 64 * (kBmPer * tid + k) + static_cast<int>(__builtin_ctzll(m));
    }
    lds_barrier();
    for (uint32_t e = tid; e < total; e += kThreads) {
      const int id = rid[e];
      const int c = count_of(e);
      if (dc) dc[id] = c;
      if (on) a.ws.exc_id[h0 + e] = id;  // (the counts stay in LDS for the gather: no exc_cnt)
    }
    if (on)
      gather_values<Tin>(a, row, h0, total, [&](uint32_t e) { return make_int2(rid[e], count_of(e)); }, rep, pres,
                         freq, ec);
  } else {
#pragma unroll
    for (int k = 0; k < kBmPer; ++k) {
      uint32_t e = pw[k];
      for (u64 m = w[k]; m; m &= m - 1) {
        const int id = 64 * (kBmPer * tid + k) + static_cast<int>(__builtin_ctzll(m));
        const int c = count_of(e);
        if (dc) dc[id] = c;
        if (on) {
          a.ws.exc_id[h0 + e] = id;
          a.ws.exc_cnt[h0 + e] = c;
        }
        ++e;
      }
    }
    // the (id, count) pairs were written by other threads of this workgroup: full barrier
    __syncthreads();
    if (on)
      gather_values<Tin>(a, row, h0, total,
                         [&](uint32_t e) { return make_int2(a.ws.exc_id[h0 + e], a.ws.exc_cnt[h0 + e]); }, rep, pres,
                         freq, ec);
  }
  *n_out = total;
  return true;
}

// Row r's penalty pass, run by a whole workgroup; `lds` is kChunk words and `red` kWaves words.
// Writes the row's exceptions to the workspace (global memory: a reader in the same workgroup
// needs a __syncthreads() first) and, up to ec.cap of them, to `ec` in LDS (visible on return).
// With dense_counts set, also writes every id's count. Returns the number of exceptions.
// *bitmap_out (when given) tells whether the penalised ids' bitmap is left in LDS from word
// kPenBitmapOffset on (bitmap_count's).
template <class Tin>
__device__ __forceinline__ uint32_t penalty_phase(const PenaltyArgs& a, int r, uint32_t* lds, uint32_t* red, ExcCache ec,
                                                  bool* bitmap_out = nullptr) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const int h0 = a.off ? a.off[r * a.hstep] : 0;
  const int h1 = a.off ? a.off[r * a.hstep + 1] : 0;
  const float rep = a.rep ? a.rep[r] : 1.0f;
  const float pres = a.pres ? a.pres[r] : 0.0f;
  const float freq = a.freq ? a.freq[r] : 0.0f;
  const bool on = (rep != 1.0f || pres != 0.0f || freq != 0.0f) && a.hist != nullptr && h1 > h0;
  const bool dense = a.dense_counts != nullptr;
  if (!on && !dense) {
    if (tid == 0) a.ws.n_exc[r] = 0;
    return 0;
  }
  const Tin* row = static_cast<const Tin*>(a.logits) + static_cast<int64_t>(r) * a.stride;
  const int32_t* hist = a.hist ? a.hist + h0 : nullptr;
  const int L = hist ? h1 - h0 : 0;
  int32_t* dc = dense ? a.dense_counts + static_cast<int64_t>(r) * a.counts_stride : nullptr;
  if (dense) {
    for (int i = tid; i < V; i += kThreads) dc[i] = 0;
    __syncthreads();  // the zeros land before the counts below overwrite some of them
  }
  uint32_t n_total = 0;
  bool bitmap = false;
  if (V <= kBmMaxV && L <= 0xFFFF && bitmap_count<Tin>(a, lds, red, ec, h0, L, V, on, dc, rep, pres, freq, row,
                                                        hist, &n_total)) {
    bitmap = true;  // (counted through a presence bitmap: two passes over the history)
  } else if (L <= kHashMaxL) {
    // ---- one pass: an (id -> count) hash table in LDS ----
    uint32_t* keys = lds;
    uint32_t* cnts = lds + kHashSlots;
    for (int i = tid; i < kHashSlots; i += kThreads) {
      keys[i] = kEmpty;
      cnts[i] = 0;
    }
    lds_barrier();
    for_each_id(hist, L, [&](int id, int) {
      if (id < 0 || id >= V) return;
      uint32_t h = (static_cast<uint32_t>(id) * 2654435761u) >> (32 - 14);  // Fibonacci hashing
      while (true) {
        const uint32_t prev = atomicCAS(&keys[h], kEmpty, static_cast<uint32_t>(id));
        if (prev == kEmpty || prev == static_cast<uint32_t>(id)) {
          atomicAdd(&cnts[h], 1u);
          break;
        }
        h = (h + 1) & (kHashSlots - 1);
      }
    });
    lds_barrier();
    // compaction: thread t owns slots 16t .. 16t + 15
    constexpr int kPer = kHashSlots / kThreads;
    uint32_t mine = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) mine += keys[tid * kPer + k] != kEmpty ? 1u : 0u;
    uint32_t e = block_excl_scan<uint32_t>(mine, red, &n_total);
    // (id, count) pairs of this thread's slots, in registers while the table is overwritten
    uint32_t sid[kPer], sc[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      sid[k] = keys[tid * kPer + k];
      sc[k] = cnts[tid * kPer + k];
    }
    lds_barrier();
    int2* stage = reinterpret_cast<int2*>(lds);  // the table is dead: stage the pairs over it
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (sid[k] == kEmpty) continue;
      if (dense) dc[sid[k]] = static_cast<int>(sc[k]);
      if (on) {
        a.ws.exc_id[h0 + e] = static_cast<int>(sid[k]);
        a.ws.exc_cnt[h0 + e] = static_cast<int>(sc[k]);
        stage[e] = make_int2(static_cast<int>(sid[k]), static_cast<int>(sc[k]));
      }
      ++e;
    }
    lds_barrier();
    if (on)
      gather_values<Tin>(a, row, h0, n_total, [&](uint32_t e) { return stage[e]; }, rep, pres, freq, ec);
  } else {
    // ---- long histories: count a window of ids at a time ----
    uint32_t* cnt = lds;
    uint32_t* present = lds + kCountWords;
    int32_t* cache = reinterpret_cast<int32_t*>(lds + kCountWords + 1024);
    const int Lc = L < kHistCache ? L : kHistCache;
    const bool wide = L > 0xFFFF;  // u16 counters hold any count of a shorter history
    const int window = wide ? kCountWords : 2 * kCountWords;
    const int nwin_words = window / 32;
    for_each_id(hist, Lc, [&](int id, int i) { cache[i] = id; });
    for (int i = tid; i < kCountWords; i += kThreads) cnt[i] = 0;
    for (int i = tid; i < 1024; i += kThreads) present[i] = 0;
    lds_barrier();
    for (int base = 0; base < V; base += window) {
      for (int i = tid; i < L; i += kThreads) {
        const int id = i < Lc ? cache[i] : hist[i];
        const unsigned rel = static_cast<unsigned>(id - base);
        if (id >= 0 && id < V && rel < static_cast<unsigned>(window)) {
          if (wide) atomicAdd(&cnt[rel], 1u);
          else atomicAdd(&cnt[rel >> 1], 1u << ((rel & 1u) << 4));
          atomicOr(&present[rel >> 5], 1u << (rel & 31u));
        }
      }
      lds_barrier();
      // thread t owns presence word t: ids base + 32t .. base + 32t + 31
      const uint32_t word = tid < nwin_words ? present[tid] : 0u;
      auto count_of = [&](int rel) -> uint32_t {
        return wide ? cnt[rel] : (cnt[rel >> 1] >> ((rel & 1) << 4)) & 0xFFFFu;
      };
      uint32_t chunk_total;
      uint32_t e = n_total + block_excl_scan<uint32_t>(__popc(word), red, &chunk_total);
      uint32_t m = word;
      while (m) {
        const int i = __ffs(m) - 1;
        m &= m - 1;
        const int id = base + 32 * tid + i;
        const int c = static_cast<int>(count_of(32 * tid + i));
        if (dense) dc[id] = c;
        if (on) {
          a.ws.exc_id[h0 + e] = id;
          a.ws.exc_cnt[h0 + e] = c;
        }
        ++e;
      }
      lds_barrier();
      // reset what this pass set: the counters of present ids and the presence words
      if (tid < nwin_words && word) {
        if (wide) {
          uint32_t mm = word;
          while (mm) {
            const int i = __ffs(mm) - 1;
            mm &= mm - 1;
            cnt[32 * tid + i] = 0;
          }
        } else {
          for (int pw = 0; pw < 16; ++pw)
            if ((word >> (2 * pw)) & 3u) cnt[16 * tid + pw] = 0;
        }
        present[tid] = 0;
      }
      n_total += chunk_total;
      lds_barrier();
    }
    // the (id, count) pairs were written by other threads of this workgroup: full barrier
    __syncthreads();
    if (on)
      gather_values<Tin>(a, row, h0, n_total,
                         [&](uint32_t e) { return make_int2(a.ws.exc_id[h0 + e], a.ws.exc_cnt[h0 + e]); }, rep, pres,
                         freq, ec);
  }
  if (tid == 0) a.ws.n_exc[r] = on ? n_total : 0u;
  if (bitmap_out) *bitmap_out = bitmap && on;
  lds_barrier();
  return on ? n_total : 0u;
}

template <class Tin>
__global__ __launch_bounds__(kThreads) void k_penalty_prep(PenaltyArgs a_) {
  const PenaltyArgs a = globalized(a_);
  __shared__ uint32_t cnt[kChunk];
  __shared__ uint32_t red[kWaves];
  penalty_phase<Tin>(a, blockIdx.x, cnt, red, ExcCache{nullptr, nullptr, 0});
}

// Penalised fp32 logits of every row: the bulk copy first, then the exceptions over it.
template <class Tin>
__global__ __launch_bounds__(kThreads) void k_penalized_out(PenaltyArgs a_, float* out_,
                                                            int64_t out_stride) {
  const PenaltyArgs a = globalized(a_);
  float* out = as_global(out_);
  const int r = blockIdx.x;
  const Tin* row = static_cast<const Tin*>(a.logits) + static_cast<int64_t>(r) * a.stride;
  float* o = out + static_cast<int64_t>(r) * out_stride;
  for (int i = threadIdx.x; i < a.V; i += kThreads) o[i] = load_one<Tin>(row, i);
  __syncthreads();
  const int h0 = a.off ? a.off[r * a.hstep] : 0;
  const uint32_t n = a.ws.n_exc[r];
  for (uint32_t e = threadIdx.x; e < n; e += kThreads) o[a.ws.exc_id[h0 + e]] = a.ws.exc_val[h0 + e];
}

}  // namespace vs
