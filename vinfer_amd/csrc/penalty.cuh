// Penalty pass: each row's token history -> exact per-id counts -> penalised logits.
//
// The penalties are not in the engine (server/protocol.py:133-135 rejects them); their
// arithmetic follows vLLM's order, one fp32 rounding per step and no fused multiply-add:
//   x = x > 0 ? x / rep : x * rep;   x = x - freq * c;   x = x - pres       (for every c > 0)
//
// Layout produced in the workspace for row r (ids with c > 0 are the row's "exceptions"):
//   n_exc[r]                         number of distinct history ids in [0, V)
//   exc_id/exc_val/exc_cnt[h0 + e]   e-th exception in ascending id order (h0 = hist_offsets[r];
//                                    a row has at most L_r exceptions, so the slots never overlap)
//   bitmap[r * nwords + w]           bit i of word w set iff id 32w + i is an exception; byte b
//                                    (little-endian) is the lane mask of the 8-id block b
#pragma once

#include "common.cuh"

namespace vs {

constexpr int kChunk = 32768;  // ids counted per LDS pass (128 KB of u32 counters)

struct Workspace {
  uint32_t* n_exc;   // [B]
  int32_t* exc_id;   // [H]
  float* exc_val;    // [H]
  int32_t* exc_cnt;  // [H]
  uint32_t* bitmap;  // [B][nwords]
  int nwords;        // ceil(V / 32)
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
  Workspace ws;
  int32_t* dense_counts;  // optional [B][counts_stride]
  int64_t counts_stride;
};

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

__device__ __forceinline__ bool row_penalized(const PenaltyArgs& a, int r) {
  const float rep = a.rep ? a.rep[r] : 1.0f;
  const float pres = a.pres ? a.pres[r] : 0.0f;
  const float freq = a.freq ? a.freq[r] : 0.0f;
  return rep != 1.0f || pres != 0.0f || freq != 0.0f;
}

// Row r's penalty pass, run by a whole workgroup; `cnt` is kChunk words of LDS and `red`
// kWaves words. Ends with the row's exceptions and bitmap written and visible to the workgroup.
template <class Tin>
__device__ void penalty_phase(const PenaltyArgs& a, int r, uint32_t* cnt, uint32_t* red) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const int h0 = a.off ? a.off[r] : 0;
  const int h1 = a.off ? a.off[r + 1] : 0;
  const bool on = row_penalized(a, r) && a.hist != nullptr && h1 > h0;
  if (!on && a.dense_counts == nullptr) {
    if (tid == 0) a.ws.n_exc[r] = 0;
    __threadfence();
    __syncthreads();
    return;
  }
  const float rep = a.rep ? a.rep[r] : 1.0f;
  const float pres = a.pres ? a.pres[r] : 0.0f;
  const float freq = a.freq ? a.freq[r] : 0.0f;
  const Tin* row = static_cast<const Tin*>(a.logits) + static_cast<int64_t>(r) * a.stride;
  const int32_t* hist = a.hist ? a.hist + h0 : nullptr;
  const int L = h1 - h0;

  uint32_t n_total = 0;
  for (int base = 0; base < V; base += kChunk) {
    for (int i = tid; i < kChunk; i += kThreads) cnt[i] = 0;
    __syncthreads();
    for (int i = tid; i < L; i += kThreads) {
      const int id = hist[i];
      const unsigned rel = static_cast<unsigned>(id - base);
      if (id >= 0 && id < V && rel < static_cast<unsigned>(kChunk)) atomicAdd(&cnt[rel], 1u);
    }
    __syncthreads();
    if (a.dense_counts) {
      int32_t* dc = a.dense_counts + static_cast<int64_t>(r) * a.counts_stride + base;
      for (int i = tid; i < kChunk && base + i < V; i += kThreads) dc[i] = static_cast<int32_t>(cnt[i]);
    }
    // Thread t owns ids base + 32t .. base + 32t + 31. Reads start at a lane-dependent offset so
    // a wave's 64 reads spread over the 32 LDS banks.
    uint32_t mask = 0;
    const int p0 = tid * 32;
#pragma unroll 8
    for (int s = 0; s < 32; ++s) {
      const int i = (s + tid) & 31;
      mask |= (cnt[p0 + i] != 0u ? 1u : 0u) << i;
    }
    const int word = (base >> 5) + tid;
    if (word < a.ws.nwords) a.ws.bitmap[static_cast<int64_t>(r) * a.ws.nwords + word] = on ? mask : 0u;
    uint32_t chunk_total;
    const uint32_t my_off = block_excl_scan<uint32_t>(__popc(mask), red, &chunk_total);
    if (on) {
      uint32_t e = n_total + my_off;
      uint32_t m = mask;
      while (m) {
        const int i = __ffs(m) - 1;
        m &= m - 1;
        const int id = base + p0 + i;
        const int c = static_cast<int>(cnt[p0 + i]);
        const float x = load_one<Tin>(row, id);
        a.ws.exc_id[h0 + e] = id;
        a.ws.exc_val[h0 + e] = apply_penalty(x, c, rep, pres, freq);
        a.ws.exc_cnt[h0 + e] = c;
        ++e;
      }
    }
    n_total += chunk_total;
    __syncthreads();
  }
  if (tid == 0) a.ws.n_exc[r] = on ? n_total : 0u;
  __threadfence();
  __syncthreads();
}

template <class Tin>
__global__ __launch_bounds__(kThreads) void k_penalty_prep(PenaltyArgs a) {
  __shared__ uint32_t cnt[kChunk];
  __shared__ uint32_t red[kWaves];
  penalty_phase<Tin>(a, blockIdx.x, cnt, red);
}

// Penalised fp32 logits of every row: the bulk copy first, then the exceptions over it.
template <class Tin>
__global__ __launch_bounds__(kThreads) void k_penalized_out(PenaltyArgs a, float* out,
                                                            int64_t out_stride) {
  const int r = blockIdx.x;
  const Tin* row = static_cast<const Tin*>(a.logits) + static_cast<int64_t>(r) * a.stride;
  float* o = out + static_cast<int64_t>(r) * out_stride;
  for (int i = threadIdx.x; i < a.V; i += kThreads) o[i] = load_one<Tin>(row, i);
  __syncthreads();
  const int h0 = a.off ? a.off[r] : 0;
  const uint32_t n = a.ws.n_exc[r];
  for (uint32_t e = threadIdx.x; e < n; e += kThreads) o[a.ws.exc_id[h0 + e]] = a.ws.exc_val[h0 + e];
}

}  // namespace vs
