// Log-probabilities of the raw logits: for each row, lp_i = x_i - M - log(sum_j exp(x_j - M))
// with M the row max (the log-softmax of the model's output, before penalties, temperature and
// filters), reported for one given token per row and for the row's n largest logits (ties by
// ascending id). The sum adds fp32 exponentials in fp64; a row whose max is not finite reports
// NaN throughout.
//
// One workgroup per row: a pass for the max and a histogram of the keys' top 13 bits, which
// gives the bin of the n-th largest key; a pass that sums the exponentials and copies every
// element of that bin and the bins above to LDS (at most kCandCap); the n-th largest key by a
// radix descent over that list, and the top n from it. A row whose top bins hold more than
// kCandCap elements (massive ties) takes the n-th key over the row and its first members in
// id order by two more passes.
//
// Tile mode (TILES, bf16 logits written by k_lm_head): the row's max and normaliser come from
// the per-tile statistics (tile max and sum of exp(x - tile max) of every 128 logits:
// S = sum_t s_t exp(m_t - M), in fp64), and the list from the tiles alone: theta, the n-th
// largest tile max, is at most the n-th largest logit (the n largest tile maxima are n logits),
// and every logit >= theta lies in a tile whose max is >= theta, so the elements >= theta of
// those tiles (n of them unless tile maxima tie) hold every logit the top n can need. A row
// with more than kTileCand such tiles takes the two passes above.
#pragma once

#include "sample.cuh"

namespace vs {

constexpr int kMaxTop = 32;     // most top logprobs per row
constexpr int kTileCand = 64;   // candidate tiles a tile-mode row reads (else two row passes)

struct LogprobArgs {
  const void* logits;  // row r at logits + r * stride
  int64_t stride;
  int V;
  const int32_t* tokens;  // [B] or null: the token whose logprob is reported
  int n_top;              // 0 .. kMaxTop
  float* out_token;       // [B] or null
  int32_t* out_top_ids;   // [B * n_top]
  float* out_top;         // [B * n_top]
  const float* tmax;      // (tile mode) [B, nT] per-tile max and sum of exp(x - max)
  const float* tsum;
  int nT;
};

// bf16 rows in one pass: the row's 16-bit key histogram (u16 counts, two keys a word) gives the
// max, the normaliser (each populated key's count times the fp32 exponential of its value, summed
// in fp64: the terms the per-element sum adds) and the n-th largest key; each thread keeps the
// three largest elements it read (packed key and position, by a min/max insertion), and those
// >= the n-th key are the candidate list, complete unless some thread's third is >= that key.
// Returns false, with no output written, for a row it does not serve -- unaligned, a NaN, an
// infinite or no finite max, a key count past 2^16, an n-th largest value <= 0 (where -0.0 and
// +0.0 would need their ties by id), an incomplete list -- and the caller runs its two passes.
// On success `kn32` is the n-th largest key as an ordered 32-bit key.
__device__ __forceinline__ bool lp_one_pass(const LogprobArgs& a, const Row<uint16_t>& row, uint32_t* hist, Cand* cand,
                                            uint32_t* sh, uint32_t* red32, u64* red64, float& M, bool& finite,
                                            double& lse, uint32_t& kn32) {
  const int tid = threadIdx.x;
  const int V = row.V;
  const int n = a.n_top;
  if (!row.vec) return false;  // (uniform)
  const int nfull = V / kBlk;
  // (a row without a whole block loads a constant block instead, unused)
  const uint4* blocks = reinterpret_cast<const uint4*>(nfull > 0 ? row.p : g_unused_block);
  // blocks tid + 1024 m; kAhead of them in flight while the previous kAhead are counted
  constexpr int kAhead = 4;
  uint4 d[kAhead];
#pragma unroll
  for (int k = 0; k < kAhead; ++k) d[k] = ld_global_u4(blocks + min(k * kThreads + tid, max(nfull - 1, 0)));
  for (int i = tid; i < 32768 / 4; i += kThreads) reinterpret_cast<uint4*>(hist)[i] = make_uint4(0, 0, 0, 0);
  if (tid < 8) sh[tid] = 0;
  __syncthreads();
  // This thread's three largest elements as packed words (key << 16 | 0xFFFF - its position
  // among the thread's elements: equal keys keep the first); the position is 8m + e for element
  // e of block tid + 1024m, and 4096 for the ragged tail's one.
  uint32_t t1 = 0, t2 = 0, t3 = 0;
  // (t1 >= t2 >= t3 throughout: the new second is the median of t1, t2 and the word, the new
  // third the median of t2, t3 and the word; v_med3_u32 takes each in one instruction)
  auto med3 = [](uint32_t a, uint32_t b, uint32_t c) {
    uint32_t d;
    asm("v_med3_u32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
  };
  auto keep = [&](uint32_t k, uint32_t pos) {
    const uint32_t pk = (k << 16) | (0xFFFFu - pos);
    const uint32_t n3 = med3(t2, t3, pk);
    t2 = med3(t1, t2, pk);
    t1 = max(t1, pk);
    t3 = n3;
  };
  const int rounds = (nfull + kAhead * kThreads - 1) / (kAhead * kThreads);  // (uniform)
  for (int it = 0; it < rounds; ++it) {
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      const int m = it * kAhead + k;
      const uint4 q = d[k];
      d[k] = ld_global_u4(blocks + min((m + kAhead) * kThreads + tid, max(nfull - 1, 0)));
      if (m * kThreads + tid < nfull) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // ordered keys of both halves at once: xor with (sign ? 0xFFFF : 0x8000)
          const uint32_t k2 = ok16x2(w[j]);
          const uint32_t klo = k2 & 0xFFFFu, khi = k2 >> 16;
          atomicAdd(&hist[klo >> 1], 1u << ((klo & 1u) << 4));
          atomicAdd(&hist[khi >> 1], 1u << ((khi & 1u) << 4));
          keep(klo, static_cast<uint32_t>(8 * m + 2 * j));
          keep(khi, static_cast<uint32_t>(8 * m + 2 * j + 1));
        }
      }
    }
  }
  for (int i = nfull * kBlk + tid; i < V; i += kThreads) {  // (fewer than kBlk elements: tid < 8)
    const uint32_t k = ok16(ld_global(row.p + i));
    atomicAdd(&hist[k >> 1], 1u << ((k & 1u) << 4));
    keep(k, 4096u);
  }
  __syncthreads();
  // the max (keys 0x0080 .. 0xFF7F are the finite values; below and above them lie -inf, +inf
  // and the NaNs)
  const uint32_t mk = static_cast<uint32_t>(block_max_u64(static_cast<u64>(t1 >> 16), red64));
  if (!(mk > 0x007Fu && mk < 0xFF80u)) return false;  // (uniform)
  M = val16(mk);
  finite = true;
  // the normaliser: words tid + 1024 i (the populated keys spread over every thread), each key's
  // count times its exponential; then the count of this thread's 64 consecutive keys (words
  // 32 tid .. 32 tid + 31)
  double s = 0.0;
  uint32_t nan = 0;
#pragma unroll 4
  for (int i = 0; i < 32; ++i) {
    const uint32_t wd = hist[tid + i * kThreads];
    if (!wd) continue;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t cnt = h ? wd >> 16 : wd & 0xFFFFu;
      const uint32_t key = 2u * (tid + i * kThreads) + h;
      if (key < 0x007Fu || key > 0xFF80u) nan += cnt;
      else if (cnt) s += static_cast<double>(cnt) * static_cast<double>(__expf(val16(key) - M));
    }
  }
  uint32_t c = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint4 v4 = reinterpret_cast<const uint4*>(hist + 32 * tid)[(q + tid) & 7];  // (rotated: banks)
    c += (v4.x & 0xFFFFu) + (v4.x >> 16) + (v4.y & 0xFFFFu) + (v4.y >> 16) + (v4.z & 0xFFFFu) + (v4.z >> 16) +
         (v4.w & 0xFFFFu) + (v4.w >> 16);
  }
  if (nan) sh[4] = 1;  // (read after the scan's barriers)
  uint32_t total;
  const uint32_t ex = block_excl_scan<uint32_t>(c, red32, &total);
  if (total != static_cast<uint32_t>(V) || sh[4]) {  // (uniform: a count wrapped, or NaNs)
    __syncthreads();  // (every thread has read the flag before the two passes reset sh)
    return false;
  }
  s = block_sum<double>(s, reinterpret_cast<double*>(red64));
  lse = static_cast<double>(M) + log(s);
  if (n <= 0) return true;
  // the n-th largest key: the wave of the thread whose keys hold it takes them, one a lane from
  // the top, and scans their counts
  const uint32_t nn = static_cast<uint32_t>(n) < static_cast<uint32_t>(V) ? static_cast<uint32_t>(n)
                                                                         : static_cast<uint32_t>(V);
  const uint32_t above = total - ex - c;  // elements in the keys above this thread's
  const u64 owner = __ballot(above < nn && nn <= above + c);
  if (owner) {  // (uniform over the wave)
    const int ol = __ffsll(static_cast<long long>(owner)) - 1;
    const uint32_t oa = __builtin_amdgcn_readlane(above, ol);
    const uint32_t key = 64u * static_cast<uint32_t>((tid & ~(kWave - 1)) + ol) + 63u - static_cast<uint32_t>(lane_id());
    const uint32_t cnt = hcount(hist, key);
    const uint32_t run = oa + wave_incl_scan<uint32_t>(cnt) - cnt;
    if (run < nn && nn <= run + cnt) {
      sh[5] = key;
      sh[7] = run + cnt;  // elements >= it
    }
  }
  __syncthreads();  // (the histogram is dead: the list goes over it)
  const uint32_t kn = sh[5];
  const bool positive = val16(kn) > 0.0f;  // (uniform)
  if (positive) {
    auto id_of = [&](uint32_t pk) -> int {
      const uint32_t pos = 0xFFFFu - (pk & 0xFFFFu);
      return pos == 4096u ? nfull * kBlk + tid : static_cast<int>(((pos >> 3) * kThreads + tid) * kBlk + (pos & 7u));
    };
    if ((t3 >> 16) >= kn && t3) sh[6] = 1;  // (this thread may hold more of them than it kept)
    if (t1 && (t1 >> 16) >= kn) cand[atomicAdd(&sh[1], 1u)] = Cand{val16(t1 >> 16), id_of(t1)};
    if (t2 && (t2 >> 16) >= kn) cand[atomicAdd(&sh[1], 1u)] = Cand{val16(t2 >> 16), id_of(t2)};
  }
  __syncthreads();
  const bool ok = positive && !sh[6] && sh[1] == sh[7];
  __syncthreads();  // (every thread has the verdict before the two passes of a fallback reset sh)
  kn32 = key_of(val16(kn));
  return ok;
}

template <class Tin, bool TILES = false>
__global__ __launch_bounds__(kThreads) void k_logprobs(LogprobArgs a) {
  constexpr int kBins = 8192;  // by the top 13 bits of the ordered key
  constexpr bool kOnePass = sizeof(Tin) == 2 && !TILES;  // (bf16 rows: one pass over a 16-bit histogram)
  __shared__ uint32_t h13[kOnePass ? 32768 : kBins];  // (then the candidate list: kCandCap 8-byte entries)
  __shared__ Radix rdx;
  __shared__ Search srch;
  __shared__ Cand top[kMaxTop];
  __shared__ uint32_t sh[8];
  static_assert(sizeof(Cand) * kCandCap <= sizeof(uint32_t) * kBins, "the candidate list fits over the bins");
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  Row<Tin> row;
  row.p = static_cast<const Tin*>(a.logits) + static_cast<int64_t>(r) * a.stride;
  row.V = a.V;
  row.nblk = (a.V + kBlk - 1) / kBlk;
  row.nstripes = (row.nblk + kThreads - 1) / kThreads;
  row.vec = (reinterpret_cast<uintptr_t>(row.p) & 15u) == 0;
  row.bm = nullptr;
  row.eid = nullptr;
  row.eval = nullptr;
  row.nexc = 0;
  const int n = a.n_top;
  if constexpr (TILES) exp_table_init();  // (published by the first barrier below)
  Cand* cand = reinterpret_cast<Cand*>(h13);
  float M = 0.0f;
  bool finite = false;
  double lse = 0.0;
  bool front = true;  // (uniform) the row passes below are needed
  if constexpr (TILES) {
    // 1. the max and the normaliser from the tile statistics (thread t: tiles t + 1024 i)
    const float* tm = a.tmax + static_cast<int64_t>(r) * a.nT;
    const float* ts = a.tsum + static_cast<int64_t>(r) * a.nT;
    float mt[4];
    uint32_t mkt = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = tid + i * kThreads;
      mt[i] = t < a.nT ? tm[t] : -INFINITY;
      const uint32_t k = key_of(mt[i]);
      mkt = k > mkt ? k : mkt;
    }
    mkt = static_cast<uint32_t>(block_max_u64(mkt, srch.red64));
    M = val_of(mkt);
    finite = mkt < key_of(INFINITY) && mkt > key_of(-INFINITY);
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = tid + i * kThreads;
      if (finite && t < a.nT && mt[i] > -INFINITY)
        s += static_cast<double>(ts[t]) * exp_nonpos(static_cast<double>(mt[i]) - static_cast<double>(M));
    }
    s = block_sum<double>(s, reinterpret_cast<double*>(srch.red64));
    lse = static_cast<double>(M) + log(s);
    if (n > 0 && a.nT >= min(n, a.V)) {
      // 2. theta (16-bit key of the n-th largest tile max), the tiles whose max is >= it, and
      // their elements >= theta into the list. (With fewer tiles than the n = min(n_top, V)
      // elements asked for, the smallest tile max need not reach the n-th largest logit: such
      // rows take the row passes below.)
      uint32_t k16[4];
      int nk = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        k16[i] = key_of(mt[i]) >> 16;  // (a bf16 value: the top half of its key; any NaN the largest)
        nk += tid + i * kThreads < a.nT;
      }
      const uint32_t nnt = static_cast<uint32_t>(min(n, a.V));
      const uint32_t th = kth_key16(k16, nk, nnt, rdx.hcnt, reinterpret_cast<uint32_t*>(rdx.hmass), sh);
      uint32_t mine = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) mine += i < nk && k16[i] >= th;
      uint32_t ntile;
      uint32_t at = block_excl_scan<uint32_t>(mine, rdx.hcnt, &ntile);
      if (ntile <= static_cast<uint32_t>(kTileCand)) {  // (uniform)
        int* ctile = reinterpret_cast<int*>(srch.tw);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (i < nk && k16[i] >= th) ctile[at++] = tid + i * kThreads;
        if (tid == 0) sh[1] = 0;
        __syncthreads();
        const uint32_t thkey = key_of(val16(th));
        // (every element's load first, then the list: kPer loads in flight per thread)
        constexpr int kPer = kTileCand * kStatTile / kThreads;
        float xs[kPer];
        int ids[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int q = tid + k * kThreads;
          ids[k] = q < static_cast<int>(ntile) * kStatTile ? ctile[q / kStatTile] * kStatTile + q % kStatTile : a.V;
          xs[k] = load_one<Tin>(row.p, ids[k] < a.V ? ids[k] : 0);
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int id = ids[k];
          const float x = xs[k];
          const bool c = id < a.V && key_of(x) >= thkey;
          const u64 bal = __ballot(c);  // (one counter update per wave round)
          if (bal) {
            const int leader = __ffsll(static_cast<long long>(bal)) - 1;
            uint32_t pos = 0;
            if (lane_id() == leader) pos = atomicAdd(&sh[1], static_cast<uint32_t>(__popcll(bal)));
            pos = __builtin_amdgcn_readlane(pos, leader) + static_cast<uint32_t>(__popcll(bal & ((1ull << lane_id()) - 1ull)));
            if (c && pos < static_cast<uint32_t>(kCandCap)) cand[pos] = Cand{x, id};
          }
        }
        front = false;
      }
    } else if (n == 0) {
      front = false;
    }
  }
  uint32_t kn32 = 0;  // (one pass) the n-th largest key, known from the histogram
  if constexpr (kOnePass) {
    if (lp_one_pass(a, row, h13, cand, sh, rdx.hcnt, srch.red64, M, finite, lse, kn32)) front = false;  // (uniform)
  }
  const bool known = kOnePass && !front;
  if (front) {
  for (int i = tid; i < kBins; i += kThreads) h13[i] = 0;
  if (tid < 8) sh[tid] = 0;
  __syncthreads();
  // 1. the max key and the bins
  uint32_t mk = 0;
  for_each_ahead(row, [&](float x, int) {
    const uint32_t k = key_of(x);
    mk = k > mk ? k : mk;
    if (n > 0) atomicAdd(&h13[k >> 19], 1u);
  });
  mk = static_cast<uint32_t>(block_max_u64(mk, srch.red64));
  const bool tiles_lse = TILES;  // (the normaliser is the tile statistics' either way)
  if (!tiles_lse) {
    M = val_of(mk);
    finite = mk < key_of(INFINITY) && mk > key_of(-INFINITY);
  }
  // the bin of the n-th largest key (thread t sums bins 8191 - 8t .. 8184 - 8t, descending)
  uint32_t bin = 0;
  if (n > 0) {
    uint32_t c8[8], s8 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c8[i] = h13[kBins - 1 - 8 * tid - i];
      s8 += c8[i];
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan<uint32_t>(s8, rdx.hcnt, &tot);
    const uint32_t nn = static_cast<uint32_t>(n) < tot ? static_cast<uint32_t>(n) : tot;
    if (nn > 0 && ex < nn && nn <= ex + s8) {
      uint32_t above = ex;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (above < nn && nn <= above + c8[i]) sh[0] = static_cast<uint32_t>(kBins - 1 - 8 * tid - i);
        above += c8[i];
      }
    }
    __syncthreads();
    bin = sh[0];
  }
  // 2. the sum of exponentials; the elements of the top bins to LDS
  double s = 0.0;
  for_each_ahead(row, [&](float x, int id) {
    if (!tiles_lse) s += static_cast<double>(__expf(x - M));
    if (n > 0) {
      const bool c = (key_of(x) >> 19) >= bin;
      const u64 bal = __ballot(c);  // (one counter update per wave round)
      if (bal) {
        const int leader = __ffsll(static_cast<long long>(bal)) - 1;
        uint32_t at = 0;
        if (lane_id() == leader) at = atomicAdd(&sh[1], static_cast<uint32_t>(__popcll(bal)));
        at = __builtin_amdgcn_readlane(at, leader) + static_cast<uint32_t>(__popcll(bal & ((1ull << lane_id()) - 1ull)));
        if (c && at < static_cast<uint32_t>(kCandCap)) cand[at] = Cand{x, id};
      }
    }
  });
  s = block_sum<double>(s, reinterpret_cast<double*>(srch.red64));
  if (!tiles_lse) lse = static_cast<double>(M) + log(s);
  }  // (front)
  auto lp = [&](float x) -> float { return finite ? static_cast<float>(static_cast<double>(x) - lse) : NAN; };
  if (tid == 0 && a.out_token && a.tokens) {
    const int t = a.tokens[r];
    a.out_token[r] = t >= 0 && t < a.V ? lp(load_one<Tin>(row.p, t)) : NAN;
  }
  if (n <= 0) return;
  // 3. the n-th largest key (with multiplicity), from the list when it holds the top bins
  __syncthreads();
  const uint32_t nc = sh[1];
  const uint32_t nn = static_cast<uint32_t>(n) < static_cast<uint32_t>(a.V) ? static_cast<uint32_t>(n)
                                                                            : static_cast<uint32_t>(a.V);
  const bool listed = nc <= static_cast<uint32_t>(kCandCap);
  const CandList cl{cand, static_cast<int>(listed ? nc : 0)};
  const uint32_t kk = known ? kn32 : listed ? radix_kth(row, &cl, nn, rdx) : radix_kth(row, nullptr, nn, rdx);
  if (known && nc <= static_cast<uint32_t>(kWave)) {  // (uniform)
    // 4/5. (one pass, a short list: every element >= the n-th key) wave 0 ranks the list by
    // descending value, then ascending id, and writes the first nn
    if (tid < kWave) {
      const bool v = static_cast<uint32_t>(tid) < nc;
      const Cand c = v ? cand[tid] : Cand{0.0f, 0};
      const uint32_t kc = key_of(c.x);
      uint32_t rank = 0;
      for (int j = 0; j < static_cast<int>(nc); ++j) {
        const Cand o = cand[j];
        const uint32_t ko = key_of(o.x);
        rank += ko > kc || (ko == kc && o.id < c.id);
      }
      if (v && rank < nn) {
        a.out_top_ids[static_cast<int64_t>(r) * n + rank] = c.id;
        a.out_top[static_cast<int64_t>(r) * n + rank] = lp(c.x);
      }
    }
  } else {
    // 4. the elements above it (fewer than nn), then the first of those equal to it by id
    if (tid == 0) sh[2] = 0;
    __syncthreads();
    if (listed) {
      for (int i = tid; i < static_cast<int>(nc); i += kThreads) {
        const Cand c = cand[i];
        if (key_of(c.x) > kk) {
          const uint32_t at = atomicAdd(&sh[2], 1u);
          if (at < static_cast<uint32_t>(kMaxTop)) top[at] = c;
        }
      }
    } else {
      for_each(row, [&](float x, int id) {
        if (key_of(x) > kk) {
          const uint32_t at = atomicAdd(&sh[2], 1u);
          if (at < static_cast<uint32_t>(kMaxTop)) top[at] = Cand{x, id};
        }
      });
    }
    __syncthreads();
    const uint32_t na = sh[2];
    const uint32_t need = nn - na;
    if (listed) {
      // a tied entry's place: the tied entries with a smaller id
      for (int i = tid; i < static_cast<int>(nc); i += kThreads) {
        const Cand c = cand[i];
        if (key_of(c.x) != kk) continue;
        uint32_t rank = 0;
        for (int j = 0; j < static_cast<int>(nc); ++j) rank += key_of(cand[j].x) == kk && cand[j].id < c.id;
        if (rank < need) top[na + rank] = c;
      }
    } else {
      // the ties' per-stripe counts, then their places stripe by stripe (ascending id)
      const int wv = tid / kWave;
      for (int j = 0; j < row.nstripes; ++j) {
        const int b = j * kThreads + tid;
        uint32_t c = 0;
        if (b < row.nblk) {
          float v[kBlk];
          const uint32_t valid = row.load(b, v);
  #pragma unroll
          for (int i = 0; i < kBlk; ++i) c += (valid >> i & 1u) && key_of(v[i]) == kk;
        }
        c = wave_sum<uint32_t>(c);
        if (lane_id() == 0) srch.cell[wv][j] = c;
      }
      __syncthreads();
      uint32_t done = 0;
      for (int j = 0; j < row.nstripes && done < need; ++j) {
        uint32_t cj = 0;
        for (int w = 0; w < kWaves; ++w) cj += static_cast<uint32_t>(srch.cell[w][j]);
        if (cj == 0) continue;  // (uniform)
        const int b = j * kThreads + tid;
        float v[kBlk];
        const uint32_t valid = b < row.nblk ? row.load(b, v) : 0u;
        uint32_t c = 0;
  #pragma unroll
        for (int i = 0; i < kBlk; ++i) c += (valid >> i & 1u) && key_of(v[i]) == kk;
        uint32_t tot;
        uint32_t at = done + block_excl_scan<uint32_t>(c, rdx.hcnt, &tot);
  #pragma unroll
        for (int i = 0; i < kBlk; ++i) {
          if ((valid >> i & 1u) && key_of(v[i]) == kk) {
            if (at < need) top[na + at] = Cand{v[i], b * kBlk + i};
            ++at;
          }
        }
        done += tot;
        __syncthreads();
      }
    }
    __syncthreads();
    // 5. order: descending value, ascending id (the ties are last, already in id order)
    if (tid < static_cast<int>(nn)) {
      const Cand c = top[tid];
      uint32_t rank = tid;
      if (tid < static_cast<int>(na)) {
        rank = 0;
        for (int j = 0; j < static_cast<int>(na); ++j) {
          const Cand o = top[j];
          rank += key_of(o.x) > key_of(c.x) || (key_of(o.x) == key_of(c.x) && o.id < c.id);
        }
      }
      a.out_top_ids[static_cast<int64_t>(r) * n + rank] = c.id;
      a.out_top[static_cast<int64_t>(r) * n + rank] = lp(c.x);
    }
  }
  for (int i = static_cast<int>(nn) + tid; i < n; i += kThreads) {  // n > V: the rest are empty
    a.out_top_ids[static_cast<int64_t>(r) * n + i] = -1;
    a.out_top[static_cast<int64_t>(r) * n + i] = -INFINITY;
  }
}

}  // namespace vs
