// Speculative-decoding verify: accept each draft token with probability min(1, p / q), where p
// and q are the target's and the draft's final probabilities of that token; at the first
// rejection, draw the replacement from the residual max(0, p - q) (renormalised); when every
// draft is accepted, the target's own draw at the position after the last draft is the bonus
// token. This is the rule of Leviathan, Kalman, Matias 2023 and Chen et al. 2023 ("speculative
// sampling"), which emits tokens distributed exactly as the target's p.
//
// Everything is decided in the sampling kernel's own fixed point, so it is exact integer
// arithmetic: a token's mass is P = rint(p~ * 2^42) (p~ = exp(z - max z) after the filters,
// 0 for dropped tokens) and its probability P / S, S the row's kept mass. Then
//   accept  <=>  m * Q_d * S_t < P_d * S_d * 2^24      (m = floor(u * 2^24))
//   residual weight of token i:  w_i = max(0, (P_i * S_d >> s) - (Q_i * S_t >> s)),
// with s = floor(log2(max(S_t, S_d))), which keeps the sum below 2^63 and each weight within a
// factor two of the target mass it stands for. The drawn token is the first id (ascending)
// whose inclusive prefix of w exceeds floor(m * R / 2^24), R the sum. A point-mass row (greedy,
// degenerate) has mass 2^42 at its token and S = 2^42.
//
// The sampling kernel has already run over every target and draft row (its RowState output
// gives each row's kept set, max and S), so this kernel reads logits only where it decides:
// the drafted tokens' two values per position, and for a rejected position the target and
// draft rows, once to sum the residual and once more inside the stripe that holds the token.
// A bf16 row holds at most 65536 distinct values, and its kept ones sit in a short run of keys
// below the row's max: the two terms of w are tabulated per key in LDS for the top kTab keys
// of each row (a kept token below that run is computed directly), so the residual pass costs
// two LDS reads per token instead of two fp64 exponentials and two 128-bit products.
#pragma once

#include <type_traits>

#include "penalty.cuh"
#include "sample.cuh"

namespace vs {

struct VerifyArgs {
  const void* tgt;  // target row (b, j), j <= K, at tgt + (b * (K + 1) + j) * tstride
  int64_t tstride;
  const void* drf;  // draft row (b, j), j < K, at drf + (b * K + j) * dstride
  int64_t dstride;
  int V, K;
  const int32_t* drafts;  // [B * K] drafted tokens
  const float* u_acc;     // [B * K] acceptance uniforms
  const float* u_res;     // [B * K] residual-draw uniforms
  const int32_t* tids;    // [B * (K + 1)] the target's draws
  const RowState* ts;     // [B * (K + 1)]
  const RowState* ds;     // [B * K]
  int32_t* out_tokens;    // [B * (K + 1)]: the emitted tokens, then -1
  int32_t* out_count;     // [B]
  int32_t* jr;            // [B] the first rejected position (K: none)
  uint32_t* done;         // [B] slices of the row's residual finished
  u64* sums;              // [B * kMaxStripes] per-stripe residual sums
  int32_t* rej;           // [B] the rejected sequences, ascending
  int32_t* nrej;          // [1] how many
  int max_slices;         // most workgroups per rejected row (a power of two)
};

using u128 = unsigned __int128;

constexpr u64 kPointMass = 4398046511104ull;  // 2^42: mass_q(1)

// A row's kept mass in the fixed point of its token masses.
__device__ __forceinline__ u64 kept_mass(const RowState& s) { return s.point >= 0 ? kPointMass : s.S; }

// Token `id` (value x) of a row: its mass under the row's state.
__device__ __forceinline__ u64 token_mass(float x, int id, const RowState& s) {
  if (s.point >= 0) return id == s.point ? kPointMass : 0;
  const bool keep = x >= s.x0 && (!s.partial || x > s.vc || (x == s.vc && id <= s.idr));
  return keep ? mass_q(ptilde(x, s.T, s.mz)) : 0;
}

// floor(u * 2^24) for u in [0, 1) (u * 2^24 is exact in fp32).
__device__ __forceinline__ u64 u24(float u) {
  const float v = u * 16777216.0f;
  return v > 0.0f ? static_cast<u64>(v) : 0ull;
}

// Order-preserving 16-bit key of a bf16 value (its bits), and the value of a key.
__device__ __forceinline__ uint32_t bf16_key(uint32_t bits) { return (bits & 0x8000u) ? (~bits & 0xFFFFu) : (bits | 0x8000u); }
// The key of a token's bf16 value for the residual's table: -0.0 takes +0.0's key (they are one
// value, and the kept set's bound `lo` is +0.0 when it is zero).
__device__ __forceinline__ uint32_t bf16_key_z(uint32_t bits) { return bf16_key(bits == 0x8000u ? 0u : bits); }
__device__ __forceinline__ float bf16_of_key(uint32_t key) {
  const uint32_t bits = (key & 0x8000u) ? (key & 0x7FFFu) : (~key & 0xFFFFu);
  return __uint_as_float(bits << 16);
}

constexpr int kTab = 8192;  // tabulated keys per row (bf16)

// One row's side of the residual: the term (mass * other_S) >> shift of each token. Both forms
// are free of branches (a point row has lo = +inf and its token in pid; other rows pid = -1),
// so that the per-token code stays one straight run.
struct ResidualSide {
  RowState st;
  u64 other_S;
  int shift;
  float lo;                // kept tokens have x >= lo (x0, or the split group's value); point row: +inf
  float vcx;               // the split group's value (partial rows), else NaN
  int pid;                 // a point row's token, else -1
  uint32_t tlo, thi;       // tabulated keys: [tlo, thi] at tab[1 + k - tlo] (tab[0] = 0)
  const u64* tab;
  u64 point_term;  // a point row's token

  __device__ __forceinline__ bool kept(float x, int id) const {
    return (x >= lo) & !((x == vcx) & (id > st.idr));
  }
  // a kept token of value x (not a point row)
  __device__ __forceinline__ u64 kept_term(float x) const {
    return static_cast<u64>((static_cast<u128>(mass_q(ptilde(x, st.T, st.mz))) * other_S) >> shift);
  }
  __device__ __forceinline__ u64 direct(float x, int id) const {
    return kept(x, id) ? kept_term(x) : (id == pid ? point_term : 0ull);
  }
  // bf16 row (not a point row) whose kept keys are all tabulated: the term of key k, value x
  // (every key >= tlo is a value >= lo, every key below maps to entry 0)
  __device__ __forceinline__ u64 term(float x, uint32_t k, int id) const {
    const int i = static_cast<int>(k) - static_cast<int>(tlo) + 1;
    const u64 t = tab[i > 0 ? i : 0];
    return ((x == vcx) & (id > st.idr)) ? 0ull : t;
  }
};

// One workgroup, a thread per sequence: the acceptance chain. Writes the accepted drafts and,
// when all are accepted, the bonus token; leaves the first rejected position in jr, clears the
// row's slice counter and lists the rejected sequences (ascending) for k_verify_residual.
template <class Tin>
__global__ __launch_bounds__(kThreads) void k_verify_accept(VerifyArgs a, int B) {
  __shared__ uint32_t red[kWaves];
  exp_table_init();
  __syncthreads();
  const int K = a.K;
  const Tin* tgt = static_cast<const Tin*>(a.tgt);
  const Tin* drf = static_cast<const Tin*>(a.drf);
  uint32_t listed = 0;
  for (int b0 = 0; b0 < B; b0 += kThreads) {
    const int b = b0 + static_cast<int>(threadIdx.x);
    int j = K;
    if (b < B) {
      for (j = 0; j < K; ++j) {
        const int d = a.drafts[b * K + j];
        if (d < 0 || d >= a.V) break;  // a token outside the vocabulary is never accepted
        const RowState st = a.ts[b * (K + 1) + j];
        const RowState sd = a.ds[b * K + j];
        const float xt = load_one<Tin>(tgt + static_cast<int64_t>(b * (K + 1) + j) * a.tstride, d);
        const float xd = load_one<Tin>(drf + static_cast<int64_t>(b * K + j) * a.dstride, d);
        const u64 P = token_mass(xt, d, st), Q = token_mass(xd, d, sd);
        const u128 lhs = static_cast<u128>(u24(a.u_acc[b * K + j])) * Q * kept_mass(st);  // < 2^127
        const u128 rhs = (static_cast<u128>(P) * kept_mass(sd)) << 24;
        if (!(lhs < rhs)) break;
      }
      int32_t* out = a.out_tokens + static_cast<int64_t>(b) * (K + 1);
      for (int i = 0; i <= K; ++i) out[i] = i < j ? a.drafts[b * K + i] : -1;
      if (j == K) {
        out[K] = a.tids[b * (K + 1) + K];
        a.out_count[b] = K + 1;
      }
      a.jr[b] = j;
      a.done[b] = 0;
    }
    const uint32_t r = j < K ? 1u : 0u;
    uint32_t tot;
    const uint32_t at = listed + block_excl_scan<uint32_t>(r, red, &tot);
    if (r) a.rej[at] = b;
    listed += tot;
  }
  if (threadIdx.x == 0) *a.nrej = static_cast<int32_t>(listed);
}

// Workgroups per rejected row: the largest power of two with every (row, slice) item on its own
// workgroup of the grid, at most max_slices.
__device__ __forceinline__ int residual_slices(int nrej, int grid, int max_slices) {
  int s = 1;
  while (2 * s <= max_slices && static_cast<int64_t>(2 * s) * nrej <= grid) s *= 2;
  return s;
}

// One (row, slice) item of the residual draw of rejected sequence b: the slice sums the residual
// over its share of the row's stripes; the last slice of the row to finish finds the stripe that
// holds floor(m * R / 2^24) and the token inside it.
template <class Tin>
__device__ __forceinline__ void residual_item(const VerifyArgs& a, int b, int slice, int slices) {
  constexpr bool kBf16 = sizeof(Tin) == 2;
  __shared__ u64 cell[kWaves][kMaxStripes];
  __shared__ u64 red[kWaves];
  __shared__ u64 tab[2][kBf16 ? kTab : 1];
  __shared__ u64 sq[4];
  __shared__ int si[4];
  const int tid = threadIdx.x;
  const int wv = tid / kWave;
  const int K = a.K;
  const int jr = a.jr[b];
  const Tin* tgt = static_cast<const Tin*>(a.tgt);
  const Tin* drf = static_cast<const Tin*>(a.drf);
  int32_t* out = a.out_tokens + static_cast<int64_t>(b) * (K + 1);
  // The rejected position's residual, over the target and draft rows at position jr.
  Row<Tin> rt, rd;
  rt.p = tgt + static_cast<int64_t>(b * (K + 1) + jr) * a.tstride;
  rd.p = drf + static_cast<int64_t>(b * K + jr) * a.dstride;
  rt.V = rd.V = a.V;
  rt.nblk = rd.nblk = (a.V + kBlk - 1) / kBlk;
  rt.nstripes = rd.nstripes = (rt.nblk + kThreads - 1) / kThreads;
  rt.vec = (reinterpret_cast<uintptr_t>(rt.p) & 15u) == 0;
  rd.vec = (reinterpret_cast<uintptr_t>(rd.p) & 15u) == 0;
  rt.bm = rd.bm = nullptr;
  rt.eid = rd.eid = nullptr;
  rt.eval = rd.eval = nullptr;
  rt.nexc = rd.nexc = 0;
  // this workgroup's stripes
  const int per = (rt.nstripes + slices - 1) / slices;
  const int j_begin = slice * per;
  const int j_end = min(rt.nstripes, j_begin + per);
  ResidualSide side[2];
  bool tabled = kBf16;
  side[0].st = a.ts[b * (K + 1) + jr];
  side[1].st = a.ds[b * K + jr];
  const u64 St = kept_mass(side[0].st), Sd = kept_mass(side[1].st);
  const int shift = 63 - __clzll(static_cast<long long>(St > Sd ? St : Sd));
  side[0].other_S = Sd;
  side[1].other_S = St;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    ResidualSide& sd = side[h];
    sd.shift = shift;
    sd.lo = sd.st.point >= 0 ? INFINITY : sd.st.partial && sd.st.vc > sd.st.x0 ? sd.st.vc : sd.st.x0;
    sd.vcx = sd.st.point < 0 && sd.st.partial ? sd.st.vc : NAN;
    sd.pid = sd.st.point >= 0 ? sd.st.point : -1;
    sd.point_term = static_cast<u64>((static_cast<u128>(kPointMass) * sd.other_S) >> shift);
    sd.tab = tab[h];
    sd.tlo = 1;
    sd.thi = 0;  // (empty)
    if constexpr (kBf16) {
      if (sd.st.point < 0) {
        // the largest finite key whose scaled value is <= the row's max (z is monotone in x)
        uint32_t lo = 0x007Fu, hi = 0xFF80u;  // -inf .. +inf
        while (lo < hi) {
          const uint32_t mid = (lo + hi + 1) / 2;
          const float x = bf16_of_key(mid);
          const float z = sd.st.T == 1.0f ? x : x / sd.st.T;
          if (z <= sd.st.mz) lo = mid;
          else hi = mid - 1;
        }
        sd.thi = lo;
        // the smallest key whose value is >= lo (lo need not be a bf16 value)
        uint32_t klo = 0x007Fu;
        if (sd.lo != -INFINITY) {
          klo = bf16_key(__float_as_uint(sd.lo) >> 16);
          if (bf16_of_key(klo) < sd.lo) ++klo;
        }
        sd.tlo = klo;
        if (sd.thi >= sd.tlo && sd.thi - sd.tlo < static_cast<uint32_t>(kTab - 1)) {
          if (tid == 0) tab[h][0] = 0;
          for (uint32_t k = sd.tlo + tid; k <= sd.thi; k += kThreads)
            tab[h][1 + k - sd.tlo] = sd.kept_term(bf16_of_key(k));  // (x >= lo: kept, but for a split group's ids)
        } else {
          tabled = false;  // (uniform) the kept keys do not fit: every term computed directly
        }
      } else {
        tabled = false;  // (uniform) a point row: its one term computed directly
      }
    }
  }
  __syncthreads();
  // The residual is 0 wherever the target drops the token (P = 0).
  const float tlo = side[0].lo;
  const int tpid = side[0].pid;
  auto kept_lanes = [&](const float (&vt)[kBlk], uint32_t valid, int blk) {
    uint32_t kept = 0;
#pragma unroll
    for (int i = 0; i < kBlk; ++i) {
      const bool k = vt[i] >= tlo || blk * kBlk + i == tpid;
      kept |= ((valid >> i) & 1u) && k ? 1u << i : 0u;
    }
    return kept;
  };
  auto weights = [&](const float (&vt)[kBlk], const float (&vd)[kBlk], uint32_t kept, int blk, u64 w[kBlk],
                     auto tab_mode) {
#pragma unroll
    for (int i = 0; i < kBlk; ++i) {
      w[i] = 0;
      if (kept & (1u << i)) {
        const int id = blk * kBlk + i;
        u64 pt, qd;
        if constexpr (decltype(tab_mode)::value) {
          pt = side[0].term(vt[i], bf16_key_z(__float_as_uint(vt[i]) >> 16), id);
          qd = side[1].term(vd[i], bf16_key_z(__float_as_uint(vd[i]) >> 16), id);
        } else {
          pt = side[0].direct(vt[i], id);
          qd = side[1].direct(vd[i], id);
        }
        w[i] = pt > qd ? pt - qd : 0;
      }
    }
  };
  // Both phases that read the rows, for one mode (tabulated terms or direct ones).
  auto residual = [&](auto tab_mode) {
    // 1. this slice's per-stripe sums; four stripes' loads of both rows in flight (the draft
    // block is read whether or not a target value in it is kept: a load behind a branch would
    // be waited for alone)
    auto stripe_sum = [&](int j, const float (&vt)[kBlk], const float (&vd)[kBlk], uint32_t valid) {
      const int blk = j * kThreads + tid;
      u64 w[kBlk];
      weights(vt, vd, kept_lanes(vt, valid, blk), blk, w, tab_mode);
      u64 s = 0;
#pragma unroll
      for (int i = 0; i < kBlk; ++i) s += w[i];
      s = wave_sum<u64>(s);
      if (lane_id() == 0) cell[wv][j - j_begin] = s;
    };
    for (int j0 = j_begin; j0 < j_end; j0 += 4) {
      if (rt.vec && rd.vec && j0 + 4 <= j_end && (j0 + 4) * kThreads * kBlk <= a.V) {
        // (uniform) four stripes wholly inside both rows
        WholeBlock<Tin> qt[4], qd[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          qt[k].load(rt.p, (j0 + k) * kThreads + tid);
          qd[k].load(rd.p, (j0 + k) * kThreads + tid);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float vt[kBlk], vd[kBlk];
          qt[k].values(vt);
          qd[k].values(vd);
          stripe_sum(j0 + k, vt, vd, 0xFFu);
        }
      } else {
        for (int j = j0; j < j_end && j < j0 + 4; ++j) {
          const int blk = j * kThreads + tid;
          float vt[kBlk], vd[kBlk];
          const uint32_t valid = blk < rt.nblk ? rt.load(blk, vt) & rd.load(blk, vd) : 0u;
          stripe_sum(j, vt, vd, valid);
        }
      }
    }
    // The stripe sums go to the other slices as relaxed agent-scope atomic stores, which are
    // coherent across the XCDs' L2s by themselves; each writer waits for its stores to complete
    // (vmcnt counts stores too) before the workgroup barrier and the counter's atomic add, and
    // the last slice loads them with agent-scope atomic loads only after that add has returned.
    // Device-scope fences (an L2 write-back and an invalidate per slice, ~15 us of a call)
    // are not needed for these few words; nothing else crosses workgroups here. This rests on
    // gfx950's encoding rather than on the HIP memory model, which orders relaxed atomics only
    // through a release/acquire pair: an agent-scope atomic store or load is a vector store or
    // load with the SC1 bit (device scope), written through the writer's L2 and read from the
    // device's coherence point, and vmcnt(0) returns once the store has reached that point.
    __syncthreads();
    if (tid < j_end - j_begin) {
      u64 t = 0;
      for (int w = 0; w < kWaves; ++w) t += cell[w][tid];
      __hip_atomic_store(&a.sums[b * kMaxStripes + j_begin + tid], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (tid == 0) si[2] = static_cast<int>(atomicAdd(&a.done[b], 1u));
    __syncthreads();
    if (si[2] != slices - 1) return;  // (uniform) another slice finishes the row
    // 2. (last slice) stripe totals; the stripe where the running sum passes floor(m * R / 2^24)
    if (wv == 0) {
      const int j = lane_id();
      const u64 t = j < rt.nstripes ? __hip_atomic_load(&a.sums[b * kMaxStripes + j], __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT)
                                    : 0ull;
      const u64 inc = wave_incl_scan<u64>(t);
      const u64 R = dpp::last(inc);
      const u64 m = u24(a.u_res[b * K + jr]);
      u64 tg = m * (R >> 24) + ((m * (R & 0xFFFFFFull)) >> 24);
      if (R > 0 && tg > R - 1) tg = R - 1;
      const bool hit = R > 0 && inc > tg && inc - t <= tg;
      const u64 hm = __ballot(hit);
      if (j == 0) {
        sq[0] = R;
        sq[1] = tg;
        si[1] = hm ? __ffsll(static_cast<long long>(hm)) - 1 : 0;
      }
      if (hit) sq[2] = inc - t;
    }
    __syncthreads();
    if (sq[0] == 0) {  // no residual mass: the target's own draw at this position
      if (tid == 0) {
        out[jr] = a.tids[b * (K + 1) + jr];
        a.out_count[b] = jr + 1;
      }
      return;
    }
    const u64 tg = sq[1];
    const int js = si[1];
    const u64 base = sq[2];
    // 3. per-thread sums inside stripe js; the thread whose block holds the target
    u64 w[kBlk] = {};
    const int blk = js * kThreads + tid;
    if (rt.vec && rd.vec && (js + 1) * kThreads * kBlk <= a.V) {  // (uniform) a whole stripe
      WholeBlock<Tin> qt, qd;
      qt.load(rt.p, blk);
      qd.load(rd.p, blk);
      float vt[kBlk], vd[kBlk];
      qt.values(vt);
      qd.values(vd);
      weights(vt, vd, kept_lanes(vt, 0xFFu, blk), blk, w, tab_mode);
    } else if (blk < rt.nblk) {
      float vt[kBlk], vd[kBlk];
      const uint32_t valid = rt.load(blk, vt) & rd.load(blk, vd);
      weights(vt, vd, kept_lanes(vt, valid, blk), blk, w, tab_mode);
    }
    u64 s = 0;
#pragma unroll
    for (int i = 0; i < kBlk; ++i) s += w[i];
    u64 tot;
    const u64 ex = block_excl_scan<u64>(s, red, &tot);
    if (s > 0 && base + ex <= tg && base + ex + s > tg) {
      // 4. this thread walks its eight lanes
      u64 c = base + ex;
      int tok = -1;
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        c += w[i];
        if (tok < 0 && w[i] > 0 && c > tg) tok = blk * kBlk + i;
      }
      out[jr] = tok;
      a.out_count[b] = jr + 1;
    }
  };
  if (kBf16 && tabled)
    residual(std::integral_constant<bool, kBf16>{});
  else
    residual(std::false_type{});
}

// The residual draws of the rejected rows: a grid of at most one workgroup per CU walks the
// (row, slice) items, row-major over the list of rejected sequences.
template <class Tin>
__global__ __launch_bounds__(kThreads) void k_verify_residual(VerifyArgs a) {
  exp_table_init();
  const int nrej = *a.nrej;
  const int slices = residual_slices(nrej, static_cast<int>(gridDim.x), a.max_slices);
  for (int item = blockIdx.x; item < nrej * slices; item += gridDim.x) {
    __syncthreads();  // (publishes the exp table; the previous item's LDS is free)
    residual_item<Tin>(a, a.rej[item / slices], item % slices, slices);
  }
}

}  // namespace vs
