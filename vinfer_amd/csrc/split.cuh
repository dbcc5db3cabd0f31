// Split rows: a small batch spreads each bf16 row over G workgroups of one launch (B * G of them
// fill the chip instead of B).
//
// Workgroup (r, g) streams slice g of row r (a contiguous range of 16-byte blocks; the last slice
// also takes the ragged tail) into an LDS histogram of the 65536 ordered 16-bit keys (u16
// counts, two per word), writes the non-empty 64-key chunks of it to its slice record (the
// chunks' 32 words each, their chunk indices and a dense map chunk -> entry; a row's values
// occupy few chunks, about 70 of 1024 for N(0, s) logits, so a record holds a few KB) and counts
// itself in at the row's arrival word. The workgroup that arrives last adds the other slices'
// records to its own histogram and finishes the row: the bf16 fast path's decisions unchanged
// (penalties, thresholds, masses, the draw's value group and member index). The drawn member is
// found in one slice: the records give each slice's count of the drawn value, so only the slice
// holding the member is searched. Nothing waits for another workgroup: the others exit after
// counting themselves in.
//
// The records cross workgroups, and XCDs, within the launch. They are written with agent-scope
// relaxed atomic stores and read with agent-scope relaxed atomic loads (`st_dev` / `ld_dev`).
// On gfx950 these are plain vector stores and loads with the SC1 bit set (device scope): a
// store is written through the writer's L2 to the device's coherence point, and a load returns
// the device-coherent copy rather than a line a reader's L2 may still hold from an earlier
// launch. Each writer waits for its own stores to complete (`s_waitcnt vmcnt(0)`) before the
// workgroup barrier that precedes the arrival's atomic, so the slice that sees the count reach
// G reads complete records. This takes the place of a release fence in every writer and an
// acquire fence in the reader, which on this GPU write back or invalidate the whole L2 of the
// XCD (the fence pair took ~6 us of each arrival). The HIP memory model alone does not promise this
// ordering for relaxed atomics; the SC1 encoding of gfx950's agent-scope atomics does.
#pragma once

#include "common.cuh"

namespace vs {

// Device-coherent stores and loads (agent-scope relaxed atomics: SC1 on gfx950), for data that
// another workgroup of the same launch reads.
template <class T>
__device__ __forceinline__ void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T ld_dev(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u4(uint4* p, uint4 v) {
  u64* q = reinterpret_cast<u64*>(p);
  st_dev<u64>(q, (static_cast<u64>(v.y) << 32) | v.x);
  st_dev<u64>(q + 1, (static_cast<u64>(v.w) << 32) | v.z);
}
__device__ __forceinline__ uint4 ld_dev_u4(const uint4* p) {
  const u64* q = reinterpret_cast<const u64*>(p);
  const u64 a = ld_dev<u64>(q), b = ld_dev<u64>(q + 1);
  return make_uint4(static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32), static_cast<uint32_t>(b),
                    static_cast<uint32_t>(b >> 32));
}

// One slice record: data[1024][32] u32 | idx[1024] u16 | emap[1024] u16 | n u32 (256-aligned).
constexpr size_t kSliceData = 0;
constexpr size_t kSliceIdx = size_t(kThreads) * 128;
constexpr size_t kSliceEmap = kSliceIdx + size_t(kThreads) * 2;
constexpr size_t kSliceN = kSliceEmap + size_t(kThreads) * 2;
constexpr size_t kSliceRecord = kSliceN + 256;
constexpr int kMaxSlices = 64;  // slices per row (the arrival word counts them in 16 bits)
constexpr uint16_t kNoEntry = 0xFFFF;
static_assert(kSliceRecord % 256 == 0, "slice records stay 256-byte aligned");

// First block of slice g (of G) of a row with nfull full 16-byte blocks.
__device__ __forceinline__ int slice_begin(int nfull, int G, int g) {
  return static_cast<int>(static_cast<int64_t>(g) * nfull / G);
}

// The keys of slice g of bf16 row `row` (V elements, 16-byte aligned) added to `hist` (65536
// u16 counts, zeroed and published by the caller). Each thread keeps eight 16-byte loads in
// flight; every thread issues them (an index past the slice rereads its last block, ignored).
__device__ __forceinline__ void slice_hist(const uint16_t* row, int V, int G, int g, uint32_t* hist) {
  const int tid = threadIdx.x;
  const int nfull = V / kBlk;
  const int b0 = slice_begin(nfull, G, g), b1 = slice_begin(nfull, G, g + 1);
  constexpr int kAhead = 8;
  uint4 q[kAhead];
  const int last = max(b1 - 1, 0);  // (the host gives every slice at least one block)
  const uint4* blocks = reinterpret_cast<const uint4*>(row);
#pragma unroll
  for (int k = 0; k < kAhead; ++k) q[k] = ld_global_u4(blocks + min(b0 + tid + k * kThreads, last));
  auto add2 = [&](uint32_t w) {
    // ordered keys of both halves at once: xor with (sign ? 0xFFFF : 0x8000)
    const uint32_t k2 = ok16x2(w);
    const uint32_t klo = k2 & 0xFFFFu, khi = k2 >> 16;
    atomicAdd(&hist[klo >> 1], 1u << ((klo & 1u) << 4));
    atomicAdd(&hist[khi >> 1], 1u << ((khi & 1u) << 4));
  };
  for (int base = b0 + tid;; base += kAhead * kThreads) {
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      if (base + k * kThreads < b1) {
        add2(q[k].x);
        add2(q[k].y);
        add2(q[k].z);
        add2(q[k].w);
      }
    }
    if (base + kAhead * kThreads >= b1) break;  // (uniform: base - tid is the same in every thread)
#pragma unroll
    for (int k = 0; k < kAhead; ++k) q[k] = ld_global_u4(blocks + min(base + (kAhead + k) * kThreads, last));
  }
  if (g == G - 1) {  // the ragged tail
    for (int i = nfull * kBlk + tid; i < V; i += kThreads) {
      const uint32_t raw = ld_global(row + i);
      const uint32_t ko = raw ^ ((raw & 0x8000u) ? 0xFFFFu : 0x8000u);
      atomicAdd(&hist[ko >> 1], 1u << ((ko & 1u) << 4));
    }
  }
}

// Writes the slice record of `hist` (complete and published by the caller's barrier) to `rec`:
// thread t takes chunk t (keys 65535 - 64t - 63 .. 65535 - 64t, words 32768 - 32t - 32 ..).
// Every store is device-coherent, and each thread waits for its stores to complete.
__device__ __forceinline__ void slice_record(const uint32_t* hist, uint8_t* rec, uint32_t* red) {
  const int tid = threadIdx.x;
  const int w0 = 32768 - 32 * tid - 32;
  uint4 c[8];
  uint32_t any = 0;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    c[s] = *reinterpret_cast<const uint4*>(&hist[w0 + 4 * s]);
    any |= c[s].x | c[s].y | c[s].z | c[s].w;
  }
  const uint32_t nz = any ? 1u : 0u;
  uint32_t n;
  const uint32_t pos = block_excl_scan<uint32_t>(nz, red, &n);
  if (nz) {
    uint4* dst = reinterpret_cast<uint4*>(rec + kSliceData) + 8 * pos;
#pragma unroll
    for (int s = 0; s < 8; ++s) st_dev_u4(dst + s, c[s]);
    st_dev<uint16_t>(reinterpret_cast<uint16_t*>(rec + kSliceIdx) + pos, static_cast<uint16_t>(tid));
  }
  st_dev<uint16_t>(reinterpret_cast<uint16_t*>(rec + kSliceEmap) + tid, nz ? static_cast<uint16_t>(pos) : kNoEntry);
  if (tid == 0) st_dev<uint32_t>(reinterpret_cast<uint32_t*>(rec + kSliceN), n);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Counts this workgroup's slice in at the row's arrival word and tells whether it is the row's
// last (then every other slice's record is complete, read with ld_dev). The word holds
// (epoch << 16 | count): a word left by another launch (another epoch, or never written)
// restarts the count at 1, so the workspace needs no clearing between launches. The last slice
// sets the count back to 0 under the same epoch, so a replay of the launch with the same
// arguments (a HIP graph keeps the epoch it was captured with) counts from 0 again. `flag` is
// an LDS word.
__device__ __forceinline__ bool slice_arrive(u64* word, u64 epoch, int G, int* flag) {
  __syncthreads();  // (every thread's record stores have completed: slice_record's vmcnt(0))
  if (threadIdx.x == 0) {
    const u64 tag = epoch & 0xFFFFFFFFFFFFull;
    u64 old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    u64 now = 0;
    // A failed exchange means another slice of this row counted itself in meanwhile: at most
    // G - 1 of them fail, so the G-th attempt succeeds.
    for (int i = 0; i < G; ++i) {
      now = (old >> 16) == tag ? old + 1 : ((tag << 16) | 1u);
      u64 seen = old;
      __hip_atomic_compare_exchange_strong(word, &seen, now, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (seen == old) break;
      old = seen;
    }
    *flag = static_cast<int>(now & 0xFFFFu);
    // (every slice of this launch has counted itself in: nothing else touches the word now)
    if ((now & 0xFFFFu) == static_cast<u64>(G)) st_dev<u64>(word, tag << 16);
  }
  __syncthreads();
  return *flag == G;
}

// (the row's last slice) Adds the other slices' records (slice `own` is already in `hist`) to
// `hist`. A unit is 16 bytes of one chunk entry (8 per entry); each thread keeps eight units'
// loads in flight. `pre` is kWave + 1 words of LDS.
__device__ __forceinline__ void slice_merge(const uint8_t* recs, int G, int own, uint32_t* hist, uint32_t* pre) {
  const int tid = threadIdx.x;
  if (tid < kWave) {
    const uint32_t n = tid < G && tid != own
                           ? ld_dev<uint32_t>(reinterpret_cast<const uint32_t*>(recs + static_cast<size_t>(tid) * kSliceRecord + kSliceN))
                           : 0u;
    const uint32_t u = 8u * n;
    const uint32_t inc = wave_incl_scan<uint32_t>(u);
    pre[tid] = inc - u;
    if (tid == kWave - 1) pre[kWave] = inc;
  }
  __syncthreads();
  const uint32_t total = pre[kWave];
  constexpr int kAhead = 8;
  for (uint32_t U0 = tid; U0 < total; U0 += kAhead * kThreads) {
    uint4 q[kAhead];
    uint32_t ch[kAhead];
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      const uint32_t U = min(U0 + k * kThreads, total - 1);
      int lo = 0, hi = G - 1;  // the slice: the last whose first unit is <= U
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pre[mid] <= U) lo = mid;
        else hi = mid - 1;
      }
      const uint32_t e = (U - pre[lo]) >> 3;
      const uint8_t* rec = recs + static_cast<size_t>(lo) * kSliceRecord;
      ch[k] = ld_dev<uint16_t>(reinterpret_cast<const uint16_t*>(rec + kSliceIdx) + e);
      q[k] = ld_dev_u4(reinterpret_cast<const uint4*>(rec + kSliceData) + 8 * e + (U & 7u));
    }
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      if (U0 + k * kThreads < total) {
        const uint32_t w = 32768u - 32u * ch[k] - 32u + 4u * ((U0 + k * kThreads) & 7u);
        if (q[k].x) atomicAdd(&hist[w], q[k].x);
        if (q[k].y) atomicAdd(&hist[w + 1], q[k].y);
        if (q[k].z) atomicAdd(&hist[w + 2], q[k].z);
        if (q[k].w) atomicAdd(&hist[w + 3], q[k].w);
      }
    }
  }
}

}  // namespace vs
