// The LM head with log-probability statistics in its epilogue: logits[b, n] = hidden[b, :] .
// W[n, :] (bf16 operands, fp32 accumulation, the result rounded to bf16 as a bf16 linear layer
// returns it; model.py:230-233 `F.linear(hidden, W)`), and for every row and every 128-column
// tile of it the max of the tile's bf16 logits and the sum of exp(x - max) over them. A later
// log-softmax (k_logprobs in tile mode) takes the row's normaliser from those statistics and
// reads only the few tiles that can hold its top n, instead of two passes over the row.
//
// MFMA tiling (gfx950, v_mfma_f32_32x32x16_bf16): a workgroup of 4 waves computes a 256 x 128
// tile of the output (all rows of a batch of up to 256) over the hidden dimension in steps of
// 64. Wave w owns rows 64w .. 64w + 63 and all 128 columns: 2 x 4 tiles of 32 x 32, 128 fp32
// accumulators per lane. Both operands are K-contiguous, so a lane's 8 bf16 of an MFMA operand
// (row l % 32, k 8 (l / 32) .. +7) are one 16-byte load: the hidden rows (2 MB at B = 256, read
// by every workgroup, so they stay in L2) come straight from global memory into registers, one
// step ahead; the weight tile, shared by the 4 waves, is staged through LDS (two buffers, rows
// padded to 144 bytes so that each 8-lane group of a 16-byte read hits distinct banks), its
// loads issued one step ahead. The weight is read once from HBM: 1.245 GB for V = 151936,
// d = 4096 -- the kernel's bound at decode batches (2 B d V flops over 2 V d bytes: B flops per
// byte, below the MFMA/HBM balance of about 312 at every B <= 256).
//
// Epilogue: the accumulators go to LDS as bf16 (a 256 x 128 tile, rows padded to 272 bytes);
// thread t then owns row t of the tile: its max and its sum of exponentials (fp32 exp of
// x - max, summed in fp32); then the tile's bf16 logits are stored 16 bytes at a time.
#pragma once

#include "common.cuh"

namespace vs {

constexpr int kLmBM = 256;         // rows per workgroup tile
constexpr int kLmBN = 128;         // columns per tile (the statistics' tile)
constexpr int kLmBK = 64;          // hidden-dimension step
constexpr int kLmThreads = 256;    // 4 waves
constexpr int kLmWStride = kLmBK + 8;   // LDS row stride of the weight tile (bf16)
constexpr int kLmOStride = kLmBN + 8;   // LDS row stride of the output tile (bf16)
constexpr int kLmWBuf = kLmBN * kLmWStride;  // bf16 per weight buffer
constexpr int kLmLds = (2 * kLmWBuf > kLmBM * kLmOStride ? 2 * kLmWBuf : kLmBM * kLmOStride) * 2;  // bytes

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

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// fp32 -> bf16, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// (one workgroup per CU: 4 waves, ~270 registers per lane with the accumulators and two steps
// of operands in flight)
__global__ __launch_bounds__(kLmThreads, 1) void k_lm_head(LmHeadArgs a) {
  __shared__ __align__(16) uint16_t lm_lds[kLmLds / 2];
  const int tid = threadIdx.x;
  const int l = lane_id();
  const int w = tid / kWave;
  const int n0 = blockIdx.x * kLmBN;
  const int m0 = blockIdx.y * kLmBM;
  const uint16_t* hid = as_global(a.hidden);
  const uint16_t* W = as_global(a.W);
  // this lane's hidden rows (one per M tile; rows past the batch read the last row, unused)
  const uint16_t* arow[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int m = min(m0 + 64 * w + 32 * mt + (l & 31), a.B - 1);
    arow[mt] = hid + static_cast<int64_t>(m) * a.ldh + 8 * (l >> 5);
  }
  // the weight tile's 16-byte chunks this thread stages: chunk q = tid + 256 c -> row q / 8,
  // part q % 8 (rows past the vocabulary read the last row, unused)
  const uint16_t* wsrc[4];
  int wdst[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int q = tid + kLmThreads * c;
    const int row = q >> 3, part = q & 7;
    wsrc[c] = W + static_cast<int64_t>(min(n0 + row, a.V - 1)) * a.ldw + 8 * part;
    wdst[c] = row * kLmWStride + 8 * part;
  }
  f32x16_t acc[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x16_t{};
  const int nk = a.d / kLmBK;
  auto load_a = [&](uint4 (&dst)[2][4], int k) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) dst[mt][ks] = ld_global_u4(reinterpret_cast<const uint4*>(arow[mt] + k + 16 * ks));
  };
  auto load_w = [&](uint4 (&dst)[4], int k) {
#pragma unroll
    for (int c = 0; c < 4; ++c) dst[c] = ld_global_u4(reinterpret_cast<const uint4*>(wsrc[c] + k));
  };
  auto store_w = [&](const uint4 (&src)[4], int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) *reinterpret_cast<uint4*>(lm_lds + buf * kLmWBuf + wdst[c]) = src[c];
  };
  // Step kt reads weight buffer kt % 2 and the hidden operands of step kt (acur); it requests
  // step kt + 1's hidden operands (anext) and step kt + 2's weight chunks (wnext: its LDS copy
  // was made one step ago), and copies step kt + 1's weight chunks (wcur, requested one step
  // ago) into the other buffer. The hidden loads go first: the wait for them at the next step
  // then does not wait for the weight loads behind them. Past the last step the indices clamp
  // (reloads, unused).
  uint4 aA[2][4], aB[2][4], wA[4], wB[4];
  load_a(aA, 0);
  load_w(wA, 0);
  load_w(wB, min(1, nk - 1) * kLmBK);
  store_w(wA, 0);
  lds_barrier();
  auto step = [&](int kt, int buf, const uint4 (&acur)[2][4], uint4 (&anext)[2][4], const uint4 (&wcur)[4],
                  uint4 (&wnext)[4]) {
    load_a(anext, min(kt + 1, nk - 1) * kLmBK);
    load_w(wnext, min(kt + 2, nk - 1) * kLmBK);
    const uint16_t* wb = lm_lds + buf * kLmWBuf;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8_t b[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        b[nt] = as_bf16x8(*reinterpret_cast<const uint4*>(wb + (32 * nt + (l & 31)) * kLmWStride + 16 * ks + 8 * (l >> 5)));
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(acur[mt][ks]), b[nt], acc[mt][nt], 0, 0, 0);
    }
    store_w(wcur, buf ^ 1);  // (every wave finished reading that buffer one step ago)
    lds_barrier();
  };
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, 0, aA, aB, wB, wA);
    if (kt + 1 < nk) step(kt + 1, 1, aB, aA, wA, wB);  // (uniform)
  }
  // ---- epilogue: the tile as bf16 in LDS (lane l, accumulator j of tile (mt, nt): row
  // 64w + 32mt + 8(j / 4) + 4(l / 32) + j % 4, column 32nt + l % 32)
  uint16_t* ot = lm_lds;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int row = 64 * w + 32 * mt + 8 * (j >> 2) + 4 * (l >> 5) + (j & 3);
        ot[row * kLmOStride + 32 * nt + (l & 31)] = static_cast<uint16_t>(bf16_rne(acc[mt][nt][j]));
      }
  lds_barrier();
  // thread t: row t of the tile -- its max and sum of exponentials over the columns inside the
  // vocabulary
  const int ncol = min(kLmBN, a.V - n0);
  {
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
  for (int q = tid; q < kLmBM * (kLmBN / 8); q += kLmThreads) {
    const int row = q >> 4, part = q & 15;
    const int m = m0 + row;
    const int c0 = 8 * part;
    if (m >= a.B || c0 >= ncol) continue;
    uint16_t* dst = out + static_cast<int64_t>(m) * a.ldo + n0 + c0;
    const uint16_t* src = ot + row * kLmOStride + c0;
    if (a.vec_out && c0 + 8 <= ncol) {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    } else {
      for (int i = 0; i < min(8, ncol - c0); ++i) dst[i] = src[i];
    }
  }
}

}  // namespace vs
