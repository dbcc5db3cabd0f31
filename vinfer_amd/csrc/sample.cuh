// Per-row sampling kernel: one 1024-thread workgroup per row.
//
// Everything is decided in the space of penalised fp32 logits x. Temperature scaling
// z = fl32(x / T) is monotone non-decreasing in x, so every filter is a threshold on x:
//   top-k  : kth largest x by radix select over ordered keys, then the smallest x whose z
//            reaches z(kth) (bisection over keys; handles division merging distinct x)
//   min-p  : the smallest x with exp(z - max z) >= min_p (fp64), by bisection over keys
//   top-p  : the cutoff value by a radix search over keys on fixed-point masses, with the
//            tokens of the cutoff value kept in ascending id order up to the exact count
// Masses are q = rint(p~ * 2^42) with p~ = exp(z - max z) in fp64, summed as integers, so every
// sum is exact and order-independent. The draw is an inverse CDF over kept tokens in ascending
// id order, found by a three-level search (stripe, thread, element) in the block-cyclic layout:
// thread t reads blocks b = j * 1024 + t (8 ids each) for stripes j = 0, 1, ...
//
// Penalised tokens ("exceptions") are masked out of the logits reads by the row's bitmap and
// visited from the exception list instead.
#pragma once

#include "common.cuh"
#include "penalty.cuh"

namespace vs {

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
  float* out_dprob;
  float* out_probs;  // probs mode when non-null
  int64_t probs_stride;
  Workspace ws;
  int has_exc;  // the workspace holds this batch's exceptions
  const int32_t* off;
  PenaltyArgs pen;  // the penalty phase's inputs (used when the kernel runs it)
};

struct Smem {
  u64 red64[kWaves];
  uint32_t red32[kWaves];
  u64 cell[kWaves][kMaxStripes];
  u64 tw[kThreads];
  uint32_t hcnt[256];
  u64 hmass[256];
  u64 slot[kBlk];
  uint32_t slot_mask;
  // broadcast scalars
  int bi[4];
  u64 bq[4];
  uint32_t bk[4];
};

template <class Tin>
struct Row {
  const Tin* p;
  int V;
  int nblk;
  int nstripes;
  bool vec;
  const uint8_t* bm;   // per-block lane masks of exceptions, or null
  const int32_t* eid;  // exceptions of this row, ascending id
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

// Visit every element of the row once: bulk lanes through `f(x, id)` in the calling thread's
// blocks, exceptions spread over the workgroup.
template <class Tin, class F>
__device__ __forceinline__ void for_each(const Row<Tin>& row, F f) {
  for (int b = threadIdx.x; b < row.nblk; b += kThreads) {
    float v[kBlk];
    const uint32_t valid = row.load(b, v);
#pragma unroll
    for (int i = 0; i < kBlk; ++i)
      if (valid & (1u << i)) f(v[i], b * kBlk + i);
  }
  for (int e = threadIdx.x; e < row.nexc; e += kThreads) f(row.eval[e], row.eid[e]);
}

// Add 1 to hist[digit] for every lane with `valid`, pre-aggregating up to four repeated digits
// per wave with ballots (the top digits of N(0, s) logits fall into a handful of bins).
__device__ __forceinline__ void hist_count(uint32_t* hist, uint32_t digit, bool valid) {
  u64 active = __ballot(valid);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    if (!active) break;
    const int leader = __ffsll(static_cast<long long>(active)) - 1;
    const uint32_t d0 = __shfl(digit, leader);
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
    const uint32_t d0 = __shfl(digit, leader);
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

// Smallest key K in [lo, hi] with pred(val_of(K)); pred(val_of(hi)) must hold.
template <class P>
__device__ uint32_t bisect_key(uint32_t lo, uint32_t hi, P pred) {
  while (lo < hi) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (pred(val_of(mid))) hi = mid;
    else lo = mid + 1;
  }
  return hi;
}

// First element index (ascending id) where the running sum of w(x, id) exceeds `target`
// (clamped to total - 1); `target = UINT64_MAX` with `u >= 0` means floor(u * total).
// Returns -1 when the total weight is 0; *total_out receives the total.
template <class Tin, class W>
__device__ int find_first(const Row<Tin>& row, W wf, u64 target, float u, Smem& s, u64* total_out) {
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  // 1. per-(wave, stripe) sums
  for (int j = 0; j < row.nstripes; ++j) {
    const int b = j * kThreads + tid;
    u64 w = 0;
    if (b < row.nblk) {
      float v[kBlk];
      const uint32_t valid = row.load(b, v);
#pragma unroll
      for (int i = 0; i < kBlk; ++i)
        if (valid & (1u << i)) w += wf(v[i], b * kBlk + i);
    }
    w = wave_sum<u64>(w);
    if (lane_id() == 0) s.cell[wv][j] = w;
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
  // 2. stripe totals, prefix over stripes, the stripe where the sum crosses the target
  if (wv == 0) {
    const int j = lane_id();
    u64 t = 0;
    if (j < row.nstripes)
      for (int w = 0; w < kWaves; ++w) t += s.cell[w][j];
    const u64 inc = wave_incl_scan<u64>(t);
    const u64 total = __shfl(inc, kWave - 1);
    u64 tg = target;
    if (u >= 0.0f) tg = static_cast<u64>(static_cast<double>(u) * static_cast<double>(total));
    if (total > 0 && tg > total - 1) tg = total - 1;
    const bool hit = total > 0 && inc > tg && (inc - t) <= tg;
    const u64 hm = __ballot(hit);
    if (j == 0) {
      s.bq[0] = total;
      s.bq[1] = tg;
      s.bi[0] = hm ? (__ffsll(static_cast<long long>(hm)) - 1) : -1;
    }
    if (hit) s.bq[2] = inc - t;  // sum before stripe j*
  }
  __syncthreads();
  const u64 total = s.bq[0];
  *total_out = total;
  if (total == 0) {
    __syncthreads();
    return -1;
  }
  const u64 tg = s.bq[1];
  const int js = s.bi[0] < 0 ? 0 : s.bi[0];
  const u64 base = s.bi[0] < 0 ? 0ull : s.bq[2];
  // 3. per-thread sums inside stripe js, prefix over threads
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

// Radix descent over ordered keys on counts: the key of the kth largest element (k >= 1).
template <class Tin>
__device__ uint32_t radix_kth(const Row<Tin>& row, uint32_t k, Smem& s) {
  uint32_t prefix = 0;
  uint32_t kk = k;
  for (int lvl = 0; lvl < 4; ++lvl) {
    const int shift = 24 - 8 * lvl;
    for (int i = threadIdx.x; i < 256; i += kThreads) s.hcnt[i] = 0;
    __syncthreads();
    const bool all = lvl == 0;
    const uint32_t pfx = prefix;
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

// Radix descent over ordered keys on masses, among elements with x >= x0: the cutoff value of
// top-p (the lowest value whose mass strictly above it is < P), its count and that mass above.
template <class Tin>
__device__ uint32_t radix_cutoff(const Row<Tin>& row, float x0, float T, float mz, double P, Smem& s,
                                 uint32_t* n_c, u64* mass_c, u64* m_above) {
  uint32_t prefix = 0;
  u64 mprev = 0;
  for (int lvl = 0; lvl < 4; ++lvl) {
    const int shift = 24 - 8 * lvl;
    for (int i = threadIdx.x; i < 256; i += kThreads) {
      s.hcnt[i] = 0;
      s.hmass[i] = 0;
    }
    __syncthreads();
    auto one = [&](float x, bool valid) {
      const uint32_t key = key_of(x);
      const bool m = valid && x >= x0 && (lvl == 0 || (key >> (shift + 8)) == prefix);
      const u64 q = m ? mass_q(ptilde(x, T, mz)) : 0ull;
      hist_mass(s.hcnt, s.hmass, (key >> shift) & 255u, q, m);
    };
    for (int b = threadIdx.x, j = 0; j < row.nstripes; ++j, b += kThreads) {
      float v[kBlk];
      uint32_t valid = b < row.nblk ? row.load(b, v) : 0u;
#pragma unroll
      for (int i = 0; i < kBlk; ++i) one(v[i], valid & (1u << i));
    }
    for (int e0 = 0; e0 < row.nexc; e0 += kThreads) {
      const int e = e0 + threadIdx.x;
      const bool ok = e < row.nexc;
      one(ok ? row.eval[e] : 0.0f, ok);
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
      for (int i = 0; i < 4; ++i) {
        if (static_cast<double>(above) < P && c[i] > 0) {
          cand = 255 - 4 * l - i;
          cand_above = above;
        }
        above += mm[i];
      }
      // lowest candidate digit = highest lane with a candidate
      const u64 hm = __ballot(cand >= 0);
      const int lw = hm ? 63 - __clzll(static_cast<long long>(hm)) : -1;
      if (l == lw) {
        s.bk[0] = static_cast<uint32_t>(cand);
        s.bq[0] = cand_above;
        s.bk[1] = c[255 - 4 * l - cand];
        s.bq[1] = mm[255 - 4 * l - cand];
      }
    }
    __syncthreads();
    prefix = (prefix << 8) | s.bk[0];
    mprev = s.bq[0];
    *n_c = s.bk[1];
    *mass_c = s.bq[1];
    __syncthreads();
  }
  *m_above = mprev;
  return prefix;
}

template <class Tin, bool PEN>
__global__ __launch_bounds__(kThreads) void k_sample(SampleArgs a) {
  __shared__ Smem s;
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int V = a.V;
  if (PEN) {
    __shared__ uint32_t cnt[kChunk];
    penalty_phase<Tin>(a.pen, r, cnt, s.red32);
  }

  Row<Tin> row;
  row.p = static_cast<const Tin*>(a.logits) + static_cast<int64_t>(r) * a.stride;
  row.V = V;
  row.nblk = (V + kBlk - 1) / kBlk;
  row.nstripes = (row.nblk + kThreads - 1) / kThreads;
  row.vec = (reinterpret_cast<uintptr_t>(row.p) & 15u) == 0;
  row.nexc = a.has_exc ? static_cast<int>(a.ws.n_exc[r]) : 0;
  if (row.nexc > 0) {
    const int h0 = a.off[r];
    row.bm = reinterpret_cast<const uint8_t*>(a.ws.bitmap + static_cast<int64_t>(r) * a.ws.nwords);
    row.eid = a.ws.exc_id + h0;
    row.eval = a.ws.exc_val + h0;
  } else {
    row.bm = nullptr;
    row.eid = nullptr;
    row.eval = nullptr;
  }

  const float T = a.temp ? a.temp[r] : 1.0f;
  const int K = a.topk ? a.topk[r] : 0;
  const float tp = a.topp ? a.topp[r] : 1.0f;
  const float mp = a.minp ? a.minp[r] : 0.0f;
  const int draft = a.draft ? a.draft[r] : -1;

  // ---- max (and first index of the max; NaN counts as the max) ----------------------------
  u64 best = 0;
  for_each(row, [&](float x, int id) {
    const u64 kq = (static_cast<u64>(key_of(x)) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(id));
    best = kq > best ? kq : best;
  });
  best = block_max_u64(best, s.red64);
  const uint32_t mkey = static_cast<uint32_t>(best >> 32);
  const int imax = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(best));
  const float xmax = val_of(mkey);

  // kept(x, id) after all filters, described by (x0, vc, idr, partial)
  float x0 = -INFINITY;
  float vc = 0.0f;
  int idr = 0;
  bool partial = false;
  int point = -1;  // greedy / degenerate rows: a point mass at this index

  const float mz = xmax / T;
  if (!(T > 0.0f) || mkey == 0xFFFFFFFFu) {
    point = imax;  // greedy (sampler.py:70-71), or a NaN logit: its first index
  } else if (mz != mz) {
    // x = +inf with T = +inf: the first index where z is NaN
    u64 tot;
    point = find_first(row, [&](float x, int) -> u64 { const float z = x / T; return z != z; }, 0ull,
                       -1.0f, s, &tot);
  } else if (mz == INFINITY) {
    u64 tot;
    point = find_first(row, [&](float x, int) -> u64 { return x / T == INFINITY; }, 0ull, -1.0f, s,
                       &tot);
  } else if (mz == -INFINITY) {
    point = 0;
  }

  if (point < 0) {
    // ---- top-k: keep z >= kth largest z (sampler.py:53-55) --------------------------------
    const uint32_t lo_key = key_of(-INFINITY);
    if (K > 0 && K < V) {
      const uint32_t kkey = radix_kth(row, static_cast<uint32_t>(K), s);
      if (tid == 0) {
        const float kz = val_of(kkey) / T;
        s.bk[2] = bisect_key(lo_key, kkey, [&](float x) { return x / T >= kz; });
      }
      __syncthreads();
      x0 = val_of(s.bk[2]);
      __syncthreads();
    }
    // ---- min-p: keep exp(z - max z) >= min_p --------------------------------------------
    if (mp > 0.0f) {
      if (tid == 0) {
        const double dmp = static_cast<double>(mp);
        s.bk[3] = bisect_key(lo_key, mkey, [&](float x) { return ptilde(x, T, mz) >= dmp; });
      }
      __syncthreads();
      const float xm = val_of(s.bk[3]);
      x0 = xm > x0 ? xm : x0;
      __syncthreads();
    }
    // ---- top-p (sampler.py:57-64) ----------------------------------------------------------
    if (tp < 1.0f) {
      u64 S0 = 0;
      for_each(row, [&](float x, int) {
        if (x >= x0) S0 += mass_q(ptilde(x, T, mz));
      });
      S0 = block_sum<u64>(S0, s.red64);
      const double P = static_cast<double>(tp) * static_cast<double>(S0);
      uint32_t nc;
      u64 massc, mabove;
      const uint32_t ck = radix_cutoff(row, x0, T, mz, P, s, &nc, &massc, &mabove);
      vc = val_of(ck);
      const u64 qc = nc ? massc / nc : 0ull;
      uint32_t rr = nc;
      if (qc > 0) {
        const double need = (P - static_cast<double>(mabove)) / static_cast<double>(qc);
        const double cr = ceil(need);
        rr = cr < 1.0 ? 1u : (cr >= static_cast<double>(nc) ? nc : static_cast<uint32_t>(cr));
      }
      if (rr >= nc) {
        x0 = vc;
      } else {
        u64 tot;
        idr = find_first(row, [&](float x, int) -> u64 { return x == vc; },
                         static_cast<u64>(rr - 1), -1.0f, s, &tot);
        partial = true;
      }
    }
  }

  auto kept = [&](float x, int id) -> bool {
    if (!(x >= x0)) return false;
    if (!partial) return true;
    return x > vc || (x == vc && id <= idr);
  };

  if (a.out_probs) {
    float* o = a.out_probs + static_cast<int64_t>(r) * a.probs_stride;
    if (point >= 0) {
      for (int i = tid; i < V; i += kThreads) o[i] = i == point ? 1.0f : 0.0f;
      return;
    }
    u64 S = 0;
    for_each(row, [&](float x, int id) {
      if (kept(x, id)) S += mass_q(ptilde(x, T, mz));
    });
    S = block_sum<u64>(S, s.red64);
    const double inv = kMassScale / static_cast<double>(S);
    for_each(row, [&](float x, int id) {
      o[id] = kept(x, id) ? static_cast<float>(ptilde(x, T, mz) * inv) : 0.0f;
    });
    return;
  }

  int tok;
  double dprob = 0.0;
  if (point >= 0) {
    tok = point;
    dprob = draft == tok ? 1.0 : 0.0;
  } else {
    const float u = a.u[r];
    u64 S;
    tok = find_first(row, [&](float x, int id) -> u64 {
      return kept(x, id) ? mass_q(ptilde(x, T, mz)) : 0ull;
    }, ~0ull, u >= 0.0f ? u : 0.0f, s, &S);
    if (draft >= 0 && draft < V && tid == 0) {
      float xd;
      const int b = draft / kBlk;
      if (row.bm && (row.bm[b] >> (draft % kBlk)) & 1u) {
        int lo = 0, hi = row.nexc - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (row.eid[mid] < draft) lo = mid + 1;
          else hi = mid;
        }
        xd = row.eval[lo];
      } else {
        xd = load_one<Tin>(row.p, draft);
      }
      if (kept(xd, draft)) dprob = ptilde(xd, T, mz) * kMassScale / static_cast<double>(S);
    }
  }
  if (tid == 0) {
    a.out_ids[r] = tok;
    if (a.out_dprob) a.out_dprob[r] = static_cast<float>(dprob);
  }
}

}  // namespace vs
