// The LM head with log-probability statistics in its epilogue: logits[b, n] = hidden[b, :] .
// W[n, :] (bf16 operands, fp32 accumulation, the result rounded to bf16 as a bf16 linear layer
// returns it; model.py:230-233 `F.linear(hidden, W)`), and for every row and every 128-column
// tile of it the max of the tile's bf16 logits and the sum of exp(x - max) over them. A later
// log-softmax (k_logprobs in tile mode) takes the row's normaliser from those statistics and
// reads only the few tiles that can hold its top n, instead of two passes over the row.
//
// MFMA tiling (gfx950, v_mfma_f32_32x32x16_bf16): a workgroup of 8 waves computes a BM x 128
// tile of the output (BM = 256: batches above 64 rows) over the hidden dimension
// in steps of 64. Both operands are K-contiguous rows, and both are staged through a ring of S
// LDS stages (BM + 128 rows of 128 bytes each) by direct global-to-LDS loads
// (global_load_lds_dwordx4: lane L of a load writes the 16 bytes at stage offset 16 L, so one
// wave-wide load fills 8 rows): no registers hold data in flight, so S - 1 steps of both
// operands are requested ahead (96 KB per CU for BM = 256) -- at decode batches the kernel
// streams the 1.245 GB weight (V = 151936, d = 4096) and is bound by HBM (2 B d V flops over
// 2 V d bytes: B flops per byte, below the MFMA/HBM balance of about 312 at every B <= 256).
// Chunk c (16 bytes) of stage row r sits at slot c ^ (r % 8): the 8 lanes of a 16-byte LDS read
// group (8 consecutive rows, one chunk) then hit 8 distinct 4-bank groups. Each wave owns a
// (32 MT) x (32 NT) block of the tile: MT x NT accumulator tiles of 16 fp32 per lane; lane l's
// MFMA operands are row l % 32, k 8 (l / 32) .. +7 of its A and B rows.
//
// Epilogue: the accumulators go to LDS as bf16 (a BM x 128 tile, rows padded to 272 bytes);
// thread t < BM then owns row t of the tile: its max and its sum of exponentials (fp32 exp of
// x - max, summed in fp32); then the tile's bf16 logits are stored 16 bytes at a time.
#pragma once

#include "common.cuh"

namespace vs {

constexpr int kLmBN = 128;       // columns per tile (the statistics' tile)
constexpr int kLmBK = 64;        // hidden-dimension step: 8 chunks of 16 bytes per row
constexpr int kLmThreads = 512;  // 8 waves
constexpr int kLmOStride = kLmBN + 8;  // LDS row stride of the output tile (bf16)

template <int BM>
struct LmTile;
template <>
struct LmTile<256> {
  static constexpr int WM = 4, MT = 2, NT = 2, S = 3;  // waves over M; tiles per wave; stages
};
template <int BM>
constexpr int lm_stage_bytes() { return (BM + kLmBN) * 128; }
template <int BM>
constexpr int lm_lds_bytes() {
  return LmTile<BM>::S * lm_stage_bytes<BM>() > BM * kLmOStride * 2 ? LmTile<BM>::S * lm_stage_bytes<BM>()
                                                                       : BM * kLmOStride * 2;
}

struct LmHeadArgs {
  const uint16_t* hidden;  // [B, d] bf16, row stride ldh (elements)
  int64_t ldh;
  const uint16_t* W;       // [V, d] bf16, row stride ldw
  int64_t ldw;
  uint16_t* logits;        // [B, V] bf16, row stride ldo
  int64_t ldo;
  float* tmax;             // [B, nT]: max of the bf16 logits of each 128-column tile
  float* tsum;             // [B, nT]: sum of exp(x - max) over the tile
  int nT;
  int B, d, V;
  int vec_out;  // logits and ldo allow 16-byte stores
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// fp32 -> bf16, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// s_waitcnt with vmcnt(n) and the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// One wave-wide global_load_lds_dwordx4: lane L's 16 bytes at `src` go to LDS byte address
// `lds` + 16 L (`lds` wave-uniform). Counted by vmcnt.
// The LDS address goes in M0, which the compiler reserves: the statement saves M0 in a scalar
// register of its own and restores it after the load has been issued, so M0 holds the
// compiler's value again when the statement ends. The s_nop is the one wait state the ISA asks
// for between an SALU write of M0 and an LDS DMA that reads it.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds) {
#if defined(__HIP_DEVICE_COMPILE__)  // (the host pass of hipcc parses device code too)
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(src)
      : "memory");
#endif
}

template <int BM>
__global__ __launch_bounds__(kLmThreads, 1) void k_lm_head(LmHeadArgs a) {
  using C = LmTile<BM>;
  constexpr int S = C::S, MT = C::MT, NT = C::NT;
  constexpr int STAGE = lm_stage_bytes<BM>();
  constexpr int PW = (BM + kLmBN) / 64;  // wave-wide loads per wave per stage (8 rows each)
  __shared__ __align__(16) uint8_t lds[lm_lds_bytes<BM>()];
  const int tid = threadIdx.x;
  const int l = lane_id();
  const int w = tid / kWave;
  const int wm = w % C::WM, wn = w / C::WM;
  const int n0 = blockIdx.x * kLmBN;
  const int m0 = blockIdx.y * BM;
  const uint16_t* hid = as_global(a.hidden);
  const uint16_t* W = as_global(a.W);
  // this lane's sources: load j of the wave fills stage rows 8 i .. 8 i + 7 (i = w + 8 j), lane
  // l the 16 bytes at slot l % 8 of row 8 i + l / 8, i.e. chunk (l % 8) ^ (l / 8) of that row
  // (rows past the batch or the vocabulary read the last one, unused)
  const uint16_t* src[PW];
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int row = 8 * (w + 8 * j) + (l >> 3);
    const int c = (l & 7) ^ (l >> 3);
    src[j] = row < BM ? hid + static_cast<int64_t>(min(m0 + row, a.B - 1)) * a.ldh + 8 * c
                      : W + static_cast<int64_t>(min(n0 + row - BM, a.V - 1)) * a.ldw + 8 * c;
  }
  const int nk = a.d / kLmBK;
  // (through inline assembly: the compiler then neither sees the loads' LDS writes nor waits for
  // them before every LDS read and barrier; the waits are the explicit ones below)
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const int wu = __builtin_amdgcn_readfirstlane(w);  // (the wave, in a scalar register: M0's operand)
  auto issue = [&](int kt) {
    const uint32_t stage = lds0 + static_cast<uint32_t>((kt % S) * STAGE);
#pragma unroll
    for (int j = 0; j < PW; ++j) lds_dma16(src[j] + kt * kLmBK, stage + 1024u * (wu + 8 * j));
  };
  f32x16_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x16_t{};
  // (a uniform number of steps in flight; the waits below take the count of loads issued after
  // the step they wait for)
#pragma unroll
  for (int s0 = 0; s0 < S - 1; ++s0)
    if (s0 < nk) issue(s0);
  const int ra0 = 32 * MT * wm + (l & 31);        // this lane's A row in its first tile
  const int rb0 = 32 * NT * wn + (l & 31);        // and its weight row
  for (int kt = 0; kt < nk; ++kt) {
    // step kt's loads are done when at most min(S - 2, nk - 1 - kt) steps' loads are in flight
    const int ahead = min(S - 2, nk - 1 - kt);  // (uniform)
    if (ahead >= 3) wait_vm<3 * PW>();
    else if (ahead == 2) wait_vm<2 * PW>();
    else if (ahead == 1) wait_vm<PW>();
    else wait_vm<0>();
    lds_barrier();  // (every wave's loads of step kt are in; every wave is done with step kt - 1)
    if (kt + S - 1 < nk) issue(kt + S - 1);  // (into step kt - 1's stage)
    const uint8_t* stage = lds + (kt % S) * STAGE;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int c = 2 * ks + (l >> 5);
      bf16x8_t av[MT], bv[NT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = ra0 + 32 * mt;
        av[mt] = as_bf16x8(*reinterpret_cast<const uint4*>(stage + r * 128 + 16 * (c ^ (r & 7))));
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int r = BM + rb0 + 32 * nt;
        bv[nt] = as_bf16x8(*reinterpret_cast<const uint4*>(stage + r * 128 + 16 * (c ^ (r & 7))));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0);
    }
  }
  lds_barrier();  // (every wave is done with the stages: the output tile goes over them)
  // ---- epilogue: the tile as bf16 in LDS (lane l, accumulator j of tile (mt, nt): row
  // 32 MT wm + 32 mt + 8 (j / 4) + 4 (l / 32) + j % 4, column 32 NT wn + 32 nt + l % 32)
  uint16_t* ot = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int row = 32 * MT * wm + 32 * mt + 8 * (j >> 2) + 4 * (l >> 5) + (j & 3);
        ot[row * kLmOStride + 32 * NT * wn + 32 * nt + (l & 31)] = static_cast<uint16_t>(bf16_rne(acc[mt][nt][j]));
      }
  lds_barrier();
  // thread t < BM: row t of the tile -- its max and sum of exponentials over the columns inside
  // the vocabulary
  const int ncol = min(kLmBN, a.V - n0);
  if (tid < BM) {
    const int m = m0 + tid;
    uint4 v[kLmBN / 8];
#pragma unroll
    for (int c = 0; c < kLmBN / 8; ++c) v[c] = *reinterpret_cast<const uint4*>(ot + tid * kLmOStride + 8 * c);
    auto lo = [](uint32_t x) { return __uint_as_float(x << 16); };
    auto hi = [](uint32_t x) { return __uint_as_float(x & 0xFFFF0000u); };
    // (the max by ordered keys: a NaN is the largest, as in the log-softmax over the row)
    uint32_t mkey = 0;
#pragma unroll
    for (int c = 0; c < kLmBN / 8; ++c) {
      const uint32_t q[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (8 * c + 2 * i < ncol) mkey = max(mkey, key_of(lo(q[i])));
        if (8 * c + 2 * i + 1 < ncol) mkey = max(mkey, key_of(hi(q[i])));
      }
    }
    const float mx = val_of(mkey);
    float s = 0.0f;
    if (mx > -INFINITY && mx < INFINITY) {  // (false for a NaN max)
#pragma unroll
      for (int c = 0; c < kLmBN / 8; ++c) {
        const uint32_t q[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (8 * c + 2 * i < ncol) s += __expf(lo(q[i]) - mx);
          if (8 * c + 2 * i + 1 < ncol) s += __expf(hi(q[i]) - mx);
        }
      }
    }
    if (m < a.B) {
      a.tmax[static_cast<int64_t>(m) * a.nT + blockIdx.x] = mx;
      a.tsum[static_cast<int64_t>(m) * a.nT + blockIdx.x] = s;
    }
  }
  // the logits: 16 chunks of 16 bytes per row (q -> row q / 16, part q % 16); rows that are not
  // 16-byte aligned, and a chunk that crosses the end of the vocabulary, element by element
  uint16_t* out = as_global(a.logits);
  for (int q = tid; q < BM * (kLmBN / 8); q += kLmThreads) {
    const int row = q >> 4, part = q & 15;
    const int m = m0 + row;
    const int c0 = 8 * part;
    if (m >= a.B || c0 >= ncol) continue;
    uint16_t* dst = out + static_cast<int64_t>(m) * a.ldo + n0 + c0;
    const uint16_t* srcp = ot + row * kLmOStride + c0;
    if (a.vec_out && c0 + 8 <= ncol) {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(srcp);
    } else {
      for (int i = 0; i < min(8, ncol - c0); ++i) dst[i] = srcp[i];
    }
  }
}

// ---- decode batches (B <= 64): the weight streamed into registers ---------------------------
// A 64-row version of the tile above (both operands through LDS) took 296-318 us at B = 8-64: each
// of its 1,187 workgroups brings the whole hidden block (64 x d) in beside its 128 weight rows,
// ~600 MB of hidden re-reads beside the 1.24 GB weight, through the same intake. Here the weight goes straight from the HBM into the
// MFMA's A operand (v_mfma_f32_16x16x32_bf16; the output computed transposed: M = vocabulary rows,
// N = batch rows), and a workgroup covers kLsRows = 640 weight rows, so that V = 151,936 takes 238
// workgroups -- one round on 256 CUs, with a fifth of the hidden re-reads (241-252 us at
// B = 8-64, d = 4096). A 256-row workgroup of 32-row waves took 323-337 us: 594 workgroups are
// 1.16 rounds of two per CU, and the second round runs on a sixth of the chip. Each of its 8 waves owns
// 80 weight rows (five 16-row tiles) and the whole 64-row batch (four 16-row tiles): 20
// accumulator tiles, 80 VGPRs, affordable at two waves per SIMD. Lane l holds row l % 16 of a
// tile at k 32 t + 8 (l / 16) .. + 7 of a 64-deep chunk (step t of two): four lanes read 64
// contiguous bytes of a row. kLsRing chunks of the weight are in flight per wave (20 KB; 160 KB a
// CU); the hidden chunk (64 rows x 128 bytes, the swizzled stage layout above, B operand: batch row
// l % 16 of a tile at the same k) rides a ring of kLsRing + 1 LDS stages filled by direct
// global-to-LDS loads, one wave-wide load per wave per chunk.
//
// Epilogue: the accumulators go to LDS as bf16, batch-major (row b: the workgroup's 640 logits of
// batch row b); thread t < 320 computes batch row t / 5's statistics over tile t % 5, and the
// logits are stored 16 bytes at a time.
constexpr int kLsThreads = 512;  // 8 waves
constexpr int kLsMT = 5;         // 16-row weight tiles per wave
constexpr int kLsRows = kLsThreads / kWave * 16 * kLsMT;  // 640: five statistics tiles
constexpr int kLsTiles = kLsRows / kLmBN;
constexpr int kLsRing = 2;       // weight chunks in flight per wave (40 VGPRs each)
constexpr int kLsStages = kLsRing + 1;
constexpr int kLsHStage = 64 * 128;        // bytes of a hidden stage: 64 rows x 64 k
constexpr int kLsOStride = kLsRows + 8;    // LDS row stride of the output staging (bf16)
constexpr int kLsLds = kLsStages * kLsHStage > 64 * kLsOStride * 2 ? kLsStages * kLsHStage : 64 * kLsOStride * 2;
static_assert(kLsRows % kLmBN == 0, "whole statistics tiles");

__global__ __launch_bounds__(kLsThreads, 1) void k_lm_stream(LmHeadArgs a) {
  __shared__ __align__(16) uint8_t lds[kLsLds];
  const int tid = threadIdx.x;
  const int l = lane_id();
  const int w = tid / kWave;
  const int nb = blockIdx.x * kLsRows;  // the workgroup's first weight row
  const int nk = a.d / kLmBK;
  // this lane's weight rows 80 w + 16 mt + l % 16 (rows past the vocabulary read the last one,
  // unused) at k 8 (l / 16) .. + 7 of each 32-deep step
  const uint4* wsrc[kLsMT];
#pragma unroll
  for (int mt = 0; mt < kLsMT; ++mt)
    wsrc[mt] = reinterpret_cast<const uint4*>(
        as_global(a.W) + static_cast<int64_t>(min(nb + 16 * kLsMT * w + 16 * mt + (l & 15), a.V - 1)) * a.ldw +
        8 * (l >> 4));
  // the hidden stage rows 8 w .. 8 w + 7 this wave fills: lane l the 16 bytes at slot l % 8 of
  // row 8 w + l / 8, i.e. chunk (l % 8) ^ (l / 8) of that row (rows past the batch read its last)
  const uint16_t* hsrc = as_global(a.hidden) + static_cast<int64_t>(min(8 * w + (l >> 3), a.B - 1)) * a.ldh +
                         8 * ((l & 7) ^ (l >> 3));
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const int wu = __builtin_amdgcn_readfirstlane(w);
  auto issue_h = [&](int kc) { lds_dma16(hsrc + kc * kLmBK, lds0 + static_cast<uint32_t>((kc % kLsStages) * kLsHStage) + 1024u * wu); };
  // q[2 mt + t]: tile mt, step t
  auto issue_w = [&](int kc, uint4 (&q)[2 * kLsMT]) {
#pragma unroll
    for (int mt = 0; mt < kLsMT; ++mt)
#pragma unroll
      for (int t = 0; t < 2; ++t) q[2 * mt + t] = wsrc[mt][kc * (kLmBK / 8) + 4 * t];
  };
  uint4 wq[kLsRing][2 * kLsMT];
  f32x4_t acc[kLsMT][4];
#pragma unroll
  for (int mt = 0; mt < kLsMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4_t{};
  // chunk c's loads: its hidden stage, then its weight (eleven per wave); chunks 0 .. kLsRing - 1
  // now. Every chunk issues the loads of chunk kc + kLsRing, of the last chunk when that is past
  // the end (unused; into registers and a stage no later chunk reads): loads on a branch would
  // make the compiler's waits before each product assume they were the latest, which waits for
  // every load in flight.
  constexpr int kPerChunk = 1 + 2 * kLsMT;
#pragma unroll
  for (int c = 0; c < kLsRing; ++c) {
    issue_h(min(c, nk - 1));
    issue_w(min(c, nk - 1), wq[c]);
  }
  // one chunk: wait for its loads (issued after them: the next kLsRing - 1 chunks' loads), the
  // barrier (every wave's hidden rows are in; every wave is done with chunk kc - 1's stage, which
  // chunk kc + kLsRing then fills), the products, and the weight of chunk kc + kLsRing into the
  // registers just used
  auto chunk = [&](int kc, uint4 (&q)[2 * kLsMT]) {
    wait_vm<kPerChunk * (kLsRing - 1)>();
    lds_barrier();
    const int next = min(kc + kLsRing, nk - 1);
    issue_h(next);
    const uint8_t* stage = lds + (kc % kLsStages) * kLsHStage;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c = 4 * t + (l >> 4);  // the hidden row's 16-byte chunk: k 8 c .. 8 c + 7 of the chunk
      bf16x8_t bv[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int r = 16 * nt + (l & 15);
        bv[nt] = as_bf16x8(*reinterpret_cast<const uint4*>(stage + r * 128 + 16 * (c ^ (r & 7))));
      }
#pragma unroll
      for (int mt = 0; mt < kLsMT; ++mt) {
        const bf16x8_t av = as_bf16x8(q[2 * mt + t]);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv[nt], acc[mt][nt], 0, 0, 0);
      }
    }
    issue_w(next, q);
  };
  static_assert(kLsRing == 2, "the chunk loop is unrolled twice");
  int kc = 0;
#pragma unroll 1
  for (; kc + 2 <= nk; kc += 2) {
    chunk(kc, wq[0]);
    chunk(kc + 1, wq[1]);
  }
  if (kc < nk) chunk(kc, wq[0]);
  wait_vm<0>();   // (the unused loads past the end, some into LDS stages, are done)
  lds_barrier();  // (every wave is done with the stages: the output goes over them)
  // ---- epilogue: lane l, accumulator j of tile (mt, nt): weight row 80 w + 16 mt + 4 (l / 16) + j,
  // batch row 16 nt + l % 16
  uint16_t* ot = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
  for (int mt = 0; mt < kLsMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ot[(16 * nt + (l & 15)) * kLsOStride + 16 * kLsMT * w + 16 * mt + 4 * (l >> 4) + j] =
            static_cast<uint16_t>(bf16_rne(acc[mt][nt][j]));
  lds_barrier();
  const int ncolw = min(kLsRows, a.V - nb);  // the workgroup's columns inside the vocabulary
  if (tid < kLsTiles * 64) {
    const int b = tid / kLsTiles, t = tid % kLsTiles;
    const int ncol = min(kLmBN, ncolw - kLmBN * t);
    if (b < a.B && ncol > 0) {
      uint4 v[kLmBN / 8];
#pragma unroll
      for (int c = 0; c < kLmBN / 8; ++c) v[c] = *reinterpret_cast<const uint4*>(ot + b * kLsOStride + kLmBN * t + 8 * c);
      auto lo = [](uint32_t x) { return __uint_as_float(x << 16); };
      auto hi = [](uint32_t x) { return __uint_as_float(x & 0xFFFF0000u); };
      // (the max by ordered keys: a NaN is the largest, as in the log-softmax over the row)
      uint32_t mkey = 0;
#pragma unroll
      for (int c = 0; c < kLmBN / 8; ++c) {
        const uint32_t q[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (8 * c + 2 * i < ncol) mkey = max(mkey, key_of(lo(q[i])));
          if (8 * c + 2 * i + 1 < ncol) mkey = max(mkey, key_of(hi(q[i])));
        }
      }
      const float mx = val_of(mkey);
      float sum = 0.0f;
      if (mx > -INFINITY && mx < INFINITY) {  // (false for a NaN max)
#pragma unroll
        for (int c = 0; c < kLmBN / 8; ++c) {
          const uint32_t q[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (8 * c + 2 * i < ncol) sum += __expf(lo(q[i]) - mx);
            if (8 * c + 2 * i + 1 < ncol) sum += __expf(hi(q[i]) - mx);
          }
        }
      }
      const int64_t at = static_cast<int64_t>(b) * a.nT + nb / kLmBN + t;
      a.tmax[at] = mx;
      a.tsum[at] = sum;
    }
  }
  // the logits: kLsRows / 8 chunks of 16 bytes per batch row; rows that are not 16-byte aligned,
  // and a chunk that crosses the end of the vocabulary, element by element
  uint16_t* out = as_global(a.logits);
  for (int q = tid; q < 64 * (kLsRows / 8); q += kLsThreads) {
    const int b = q / (kLsRows / 8), c0 = 8 * (q % (kLsRows / 8));
    if (b >= a.B || c0 >= ncolw) continue;
    uint16_t* dst = out + static_cast<int64_t>(b) * a.ldo + nb + c0;
    const uint16_t* srcp = ot + b * kLsOStride + c0;
    if (a.vec_out && c0 + 8 <= ncolw) {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(srcp);
    } else {
      for (int i = 0; i < min(8, ncolw - c0); ++i) dst[i] = srcp[i];
    }
  }
}

// ---- the tile statistics of logits from another GEMM ----------------------------------------
// What the epilogues above write beside their own logits, for bf16 logits another GEMM wrote
// (above 64 rows the library's GEMM beats the MFMA tiles above): per row and kLmBN logits, the
// max (ordered keys: a NaN is the largest) and the fp32 sum of exp(x - max) over the tile (0 when
// the max is infinite or NaN). Sixteen lanes a tile, eight logits a lane (a lane's max by IEEE
// maximum, its ordered keys only when a NaN is among them), 16-lane DPP reductions (the sum in
// another order than an epilogue's, so it may differ in the last bits); grid (ceil(nT / 16), B)
// of 256-thread workgroups.
constexpr int kTsThreads = 256;
__global__ __launch_bounds__(kTsThreads) void k_tile_stats(const uint16_t* logits, int64_t stride, int V, int nT,
                                                           float* tmax, float* tsum) {
  const int r = blockIdx.y;
  const int l16 = threadIdx.x & 15;
  const int t = blockIdx.x * (kTsThreads / 16) + static_cast<int>(threadIdx.x >> 4);  // (the same in a 16-lane row)
  const uint16_t* row = as_global(logits) + static_cast<int64_t>(r) * stride;
  const int i0 = t * kLmBN + 8 * l16;  // this lane's first logit
  float x[8];
  int nv = 0;  // this lane's logits inside the row
  if (t < nT) {
    if ((reinterpret_cast<uintptr_t>(row + i0) & 15u) == 0 && i0 + 8 <= V) {
      const uint4 q = ld_global_u4(reinterpret_cast<const uint4*>(row + i0));
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      }
      nv = 8;
    } else {
      nv = max(0, min(8, V - i0));
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = i < nv ? bf16_to_f32(ld_global(row + i0 + i)) : 0.0f;
    }
  }
  uint32_t mk = 0;  // (below every key)
  auto key_max = [&](int n) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < n) mk = max(mk, key_of(x[i]));
  };
  if (nv == 8) {
    // the IEEE maximum of the eight (four three-operand maxima; -0 below +0, as in key order): the
    // value of the largest key unless one of them is a NaN, which makes it a NaN -- then the keys
    // decide which NaN
    float bx = x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) bx = __builtin_elementwise_maximum(bx, x[i]);
    mk = key_of(bx);
    if (bx != bx) {
      mk = 0;
      key_max(8);
    }
  } else {
    key_max(nv);
  }
  auto umax = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  mk = umax(mk, dpp::mov<dpp::kXor1>(mk));
  mk = umax(mk, dpp::mov<dpp::kXor2>(mk));
  mk = umax(mk, dpp::mov<dpp::kHalfMirror>(mk));
  mk = umax(mk, dpp::mov<dpp::kMirror>(mk));
  const float mx = val_of(mk);
  float s = 0.0f;
  if (mx > -INFINITY && mx < INFINITY) {  // (false for a NaN max)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < nv) s += __expf(x[i] - mx);
  }
  auto fadd = [](float a, uint32_t b) { return a + __uint_as_float(b); };
  s = fadd(s, dpp::mov<dpp::kXor1>(__float_as_uint(s)));
  s = fadd(s, dpp::mov<dpp::kXor2>(__float_as_uint(s)));
  s = fadd(s, dpp::mov<dpp::kHalfMirror>(__float_as_uint(s)));
  s = fadd(s, dpp::mov<dpp::kMirror>(__float_as_uint(s)));
  if (t < nT && l16 == 0) {
    as_global(tmax)[static_cast<int64_t>(r) * nT + t] = mx;
    as_global(tsum)[static_cast<int64_t>(r) * nT + t] = s;
  }
}

// ---- a few batch rows: matrix-vector products -------------------------------------------------
// At B <= 4 the 64-row tile above loads 60 or more rows of padding beside each step's weight (a
// CU's intake, not the HBM, bounds the kernel), so these batches take a kernel of their own:
// each workgroup computes one 128-column statistics tile for every row, each wave 16 of its
// weight rows. Lane l holds chunks l + 64 c (c < CPL, d = 512 CPL) of the NB hidden rows in
// registers and reads the same chunks of each weight row with plain 16-byte loads, a window of
// rows ahead; a logit is the lanes' fp32 sums of bf16 pair products (v_dot2) added over the
// wave. The epilogue is each row's tile statistics and bf16 logits, as above.
constexpr int kGvThreads = 512;  // 8 waves, 16 weight rows each
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot8(uint4 w, uint4 h, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, h.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, h.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, h.z), acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, h.w), acc, false);
}

// NB hidden rows (B <= NB; rows past the batch repeat its last row, unused)
template <int CPL, int NB>
__global__ __launch_bounds__(kGvThreads, 1) void k_lm_gemv(LmHeadArgs a) {
  constexpr int kRowsPerWave = kLmBN / (kGvThreads / kWave);  // 16
  constexpr int kRing = NB == 1 ? 4 : 2;  // weight rows in flight per wave (registers: hidden + ring)
  static_assert(kRowsPerWave % kRing == 0, "whole groups of rows");
  __shared__ float lg[NB][kLmBN];  // the tile's logits, rounded to bf16
  const int l = lane_id();
  const int w = threadIdx.x / kWave;
  const int n0 = blockIdx.x * kLmBN;
  uint4 hv[NB][CPL];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint4* hid = reinterpret_cast<const uint4*>(as_global(a.hidden) + static_cast<int64_t>(min(b, a.B - 1)) * a.ldh);
#pragma unroll
    for (int c = 0; c < CPL; ++c) hv[b][c] = hid[l + 64 * c];
  }
  // row i of this wave: n0 + kRowsPerWave w + i (rows past the vocabulary read the last one)
  auto load_row = [&](int i, uint4 (&dst)[CPL]) {
    const uint4* r = reinterpret_cast<const uint4*>(
        as_global(a.W) + static_cast<int64_t>(min(n0 + kRowsPerWave * w + i, a.V - 1)) * a.ldw);
#pragma unroll
    for (int c = 0; c < CPL; ++c) dst[c] = r[l + 64 * c];
  };
  // a rolling window: slot k holds row kRing g + k and is reloaded with the next group's row as
  // soon as its dot products are taken (the last group, peeled, reloads nothing)
  uint4 rb[kRing][CPL];
#pragma unroll
  for (int k = 0; k < kRing; ++k) load_row(k, rb[k]);
  auto group = [&](int g, bool reload) {
#pragma unroll
    for (int k = 0; k < kRing; ++k) {
      float s[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          if (c & 1) s1 = dot8(rb[k][c], hv[b][c], s1);
          else s0 = dot8(rb[k][c], hv[b][c], s0);
        }
        s[b] = s0 + s1;
      }
      if (reload) load_row(kRing * (g + 1) + k, rb[k]);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float v = wave_sum<float>(s[b]);
        if (l == 0) lg[b][kRowsPerWave * w + kRing * g + k] = __uint_as_float(bf16_rne(v) << 16);
      }
    }
  };
#pragma unroll 1
  for (int g = 0; g < kRowsPerWave / kRing - 1; ++g) group(g, true);
  group(kRowsPerWave / kRing - 1, false);
  __syncthreads();
  if (w >= NB || w >= a.B) return;
  // wave b < B: row b's statistics over the columns inside the vocabulary (lane l: columns l,
  // l + 64), then its bf16 logits, 16 bytes per lane
  const int b = w;
  const int ncol = min(kLmBN, a.V - n0);
  const float x0 = lg[b][l], x1 = lg[b][l + 64];
  uint32_t mk = 0;
  if (l < ncol) mk = key_of(x0);
  if (l + 64 < ncol) mk = max(mk, key_of(x1));
  mk = dpp::reduce(mk, [](uint32_t p, uint32_t q) { return p > q ? p : q; });
  const float mx = val_of(mk);
  float e = 0.0f;
  if (mx > -INFINITY && mx < INFINITY) {  // (false for a NaN max)
    if (l < ncol) e += __expf(x0 - mx);
    if (l + 64 < ncol) e += __expf(x1 - mx);
  }
  e = wave_sum<float>(e);
  if (l == 0) {
    a.tmax[static_cast<int64_t>(b) * a.nT + blockIdx.x] = mx;
    a.tsum[static_cast<int64_t>(b) * a.nT + blockIdx.x] = e;
  }
  uint16_t* out = as_global(a.logits) + static_cast<int64_t>(b) * a.ldo + n0;
  const int c0 = 8 * l;
  if (l < kLmBN / 8 && c0 < ncol) {
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      q[i] = (__float_as_uint(lg[b][c0 + 2 * i]) >> 16) | (__float_as_uint(lg[b][c0 + 2 * i + 1]) & 0xFFFF0000u);
    if (a.vec_out && c0 + 8 <= ncol) {
      *reinterpret_cast<uint4*>(out + c0) = make_uint4(q[0], q[1], q[2], q[3]);
    } else {
      for (int i = 0; i < min(8, ncol - c0); ++i) out[c0 + i] = static_cast<uint16_t>(i & 1 ? q[i / 2] >> 16 : q[i / 2] & 0xFFFFu);
    }
  }
}

}  // namespace vs
