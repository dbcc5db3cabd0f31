// The draw's uniform of (seed, position), for many rows per call: host code (vsamp_uniforms), and
// the same functions compiled for the device (vsamp_uniforms_device, for loops whose steps are
// replayed from a captured graph and cannot run host code between them).
//
// position_seed(seed, position) is BLAKE2b with an 8-byte digest of the ASCII text
// "<seed>:<position>", read little-endian, top bit cleared (src/vinfer/runtime/sampler.py:44-47).
// BLAKE2b here follows RFC 7693 (unkeyed, one 128-byte block: the text is at most 41 bytes,
// built into registers: no byte array, so the device code needs no scratch memory).
// The uniform is then the top 24 bits of the SplitMix64 output function (Steele, Lea, Flood
// 2014) of that seed, times 2^-24: a multiple of 2^-24 in [0, 1), exact in fp32.
#pragma once

#include <cstdint>

namespace vs_host {

#define VS_HD __host__ __device__ __forceinline__

constexpr uint64_t kBlakeIV[8] = {0x6A09E667F3BCC908ull, 0xBB67AE8584CAA73Bull, 0x3C6EF372FE94F82Bull,
                                  0xA54FF53A5F1D36F1ull, 0x510E527FADE682D1ull, 0x9B05688C2B3E6C1Full,
                                  0x1F83D9ABFB41BD6Bull, 0x5BE0CD19137E2179ull};

// Message word schedule of the ten distinct rounds (RFC 7693, section 2.7); round i uses row i % 10.
constexpr uint8_t kSigma[10][16] = {
    {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15}, {14, 10, 4, 8, 9, 15, 13, 6, 1, 12, 0, 2, 11, 7, 5, 3},
    {11, 8, 12, 0, 5, 2, 15, 13, 10, 14, 3, 6, 7, 1, 9, 4}, {7, 9, 3, 1, 13, 12, 11, 14, 2, 6, 5, 10, 4, 0, 15, 8},
    {9, 0, 5, 7, 2, 4, 10, 15, 14, 1, 11, 12, 6, 8, 3, 13}, {2, 12, 6, 10, 0, 11, 8, 3, 4, 13, 7, 5, 15, 14, 1, 9},
    {12, 5, 1, 15, 14, 13, 4, 10, 0, 7, 6, 3, 9, 2, 8, 11}, {13, 11, 7, 14, 12, 1, 3, 9, 5, 0, 15, 4, 8, 6, 2, 10},
    {6, 15, 14, 9, 11, 3, 0, 8, 12, 2, 13, 7, 1, 4, 10, 5}, {10, 2, 8, 4, 7, 6, 1, 5, 15, 11, 9, 14, 3, 12, 13, 0},
};

// x rotated right by n (0 < n < 64, a constant once inlined). The device pass writes it as two
// funnel shifts of the 32-bit halves (v_alignbit_b32; a rotation by 32 swaps them), which the
// compiler does not form from the 64-bit expression.
VS_HD uint64_t rotr64(uint64_t x, int n) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t lo = static_cast<uint32_t>(x), hi = static_cast<uint32_t>(x >> 32);
  uint32_t nl, nh;
  if (n == 32) {
    nl = hi;
    nh = lo;
  } else if (n < 32) {
    nl = __builtin_amdgcn_alignbit(hi, lo, n);
    nh = __builtin_amdgcn_alignbit(lo, hi, n);
  } else {
    nl = __builtin_amdgcn_alignbit(lo, hi, n - 32);
    nh = __builtin_amdgcn_alignbit(hi, lo, n - 32);
  }
  return (static_cast<uint64_t>(nh) << 32) | nl;
#else
  return (x >> n) | (x << (64 - n));
#endif
}

VS_HD void blake_mix(uint64_t* v, int a, int b, int c, int d, uint64_t x, uint64_t y) {
  v[a] = v[a] + v[b] + x;
  v[d] = rotr64(v[d] ^ v[a], 32);
  v[c] = v[c] + v[d];
  v[b] = rotr64(v[b] ^ v[c], 24);
  v[a] = v[a] + v[b] + y;
  v[d] = rotr64(v[d] ^ v[a], 16);
  v[c] = v[c] + v[d];
  v[b] = rotr64(v[b] ^ v[c], 63);
}

// The first 8 bytes (little-endian) of the 8-byte BLAKE2b digest of a text of n <= 48 bytes held
// as six little-endian words (zero past the text). The loops are unrolled: the tables are then
// indexed by constants and the message words are registers, on the device too.
VS_HD uint64_t blake2b_8(const uint64_t (&t)[6], int n) {
  uint64_t m[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) m[i] = i < 6 ? t[i] : 0ull;
  uint64_t h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = kBlakeIV[i];
  h[0] ^= 0x01010000ull ^ 8ull;  // depth 1, fanout 1, no key, 8-byte digest
  uint64_t v[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = h[i];
    v[i + 8] = kBlakeIV[i];
  }
  v[12] ^= static_cast<uint64_t>(n);  // bytes compressed (the high counter word stays 0)
  v[14] = ~v[14];                     // the last block
#pragma unroll
  for (int r = 0; r < 12; ++r) {
    const uint8_t* s = kSigma[r % 10];
    blake_mix(v, 0, 4, 8, 12, m[s[0]], m[s[1]]);
    blake_mix(v, 1, 5, 9, 13, m[s[2]], m[s[3]]);
    blake_mix(v, 2, 6, 10, 14, m[s[4]], m[s[5]]);
    blake_mix(v, 3, 7, 11, 15, m[s[6]], m[s[7]]);
    blake_mix(v, 0, 5, 10, 15, m[s[8]], m[s[9]]);
    blake_mix(v, 1, 6, 11, 12, m[s[10]], m[s[11]]);
    blake_mix(v, 2, 7, 8, 13, m[s[12]], m[s[13]]);
    blake_mix(v, 3, 4, 9, 14, m[s[14]], m[s[15]]);
  }
  return h[0] ^ v[0] ^ v[8];
}

constexpr uint64_t kPow10[20] = {1ull, 10ull, 100ull, 1000ull, 10000ull, 100000ull, 1000000ull, 10000000ull,
                                 100000000ull, 1000000000ull, 10000000000ull, 100000000000ull, 1000000000000ull,
                                 10000000000000ull, 100000000000000ull, 1000000000000000ull, 10000000000000000ull,
                                 100000000000000000ull, 1000000000000000000ull, 10000000000000000000ull};

// ---- the decimal text "<seed>:<position>" as little-endian message words ---------------------
// Built without per-character placement: each number's digits come from three base-10^8 parts
// (two 64-bit divisions by a constant, then 32-bit ones), as twenty ASCII digits with leading
// zeros in five little-endian 32-bit words (byte 0 = the most significant digit); the leading
// zeros are dropped by one variable shift, and the parts are placed at their byte offsets by
// variable shifts of the whole message.

// The eight ASCII digits of v < 10^8 (leading zeros kept), most significant first in byte order:
// lo = bytes 0-3, hi = bytes 4-7.
VS_HD void ascii8(uint32_t v, uint32_t& lo, uint32_t& hi) {
  uint32_t d[8];
#pragma unroll
  for (int k = 7; k >= 0; --k) {  // k = 7: the units digit
    const uint32_t q = v / 10u;
    d[k] = v - 10u * q;
    v = q;
  }
  lo = d[0] | (d[1] << 8) | (d[2] << 16) | (d[3] << 24) | 0x30303030u;
  hi = d[4] | (d[5] << 8) | (d[6] << 16) | (d[7] << 24) | 0x30303030u;
}

// The decimal text of x (no leading zeros; "0" for 0) in five little-endian words, zero past its
// end; returns its length (1 .. 20).
VS_HD int decimal_text(uint64_t x, uint32_t (&t)[5]) {
  const uint64_t q = x / 100000000u;
  const uint32_t r0 = static_cast<uint32_t>(x - q * 100000000u);
  const uint32_t q2 = static_cast<uint32_t>(q / 100000000u);  // < 1845
  const uint32_t r1 = static_cast<uint32_t>(q - static_cast<uint64_t>(q2) * 100000000u);
  uint32_t s[6];  // the 20 digits at bytes 4 .. 23 of s (bytes 0 .. 3 unused, zero)
  uint32_t top_lo, top_hi;
  ascii8(q2, top_lo, top_hi);  // (its first four digits are zeros)
  s[0] = 0;
  s[1] = top_hi;
  ascii8(r1, s[2], s[3]);
  ascii8(r0, s[4], s[5]);
  int n = 1;
#pragma unroll
  for (int k = 1; k < 20; ++k) n += x >= kPow10[k] ? 1 : 0;
  // drop the 20 - n leading zeros: the text starts at byte 24 - n of s
  const int z = 24 - n;
  const int wz = z >> 2, bz = 8 * (z & 3);
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    uint32_t a = 0, b = 0;  // words wz + i and wz + i + 1 of s (zero past the end)
#pragma unroll
    for (int j = 1; j < 6; ++j) {
      a = wz + i == j ? s[j] : a;
      b = wz + i + 1 == j ? s[j] : b;
    }
    t[i] = static_cast<uint32_t>(((static_cast<uint64_t>(b) << 32) | a) >> bz);
  }
  return n;
}

// m (twelve little-endian words, the 48-byte message) |= the 20-byte string x placed at byte
// offset o (0 <= o <= 28).
VS_HD void place(uint32_t (&m)[12], const uint32_t (&x)[5], int o) {
  const int bo = 8 * (o & 3);
  uint32_t y[12];
  // the byte shift within words
#pragma unroll
  for (int j = 0; j < 12; ++j) {
    const uint32_t hi = j < 5 ? x[j] : 0u, lo = j >= 1 && j - 1 < 5 ? x[j - 1] : 0u;
    y[j] = static_cast<uint32_t>(((static_cast<uint64_t>(hi) << 32) | lo) >> (32 - bo));
  }
  // the word shift, o / 4 = 4 a + 2 b + c words, by halving steps
  const int wo = o >> 2;
#pragma unroll
  for (int step = 4; step >= 1; step >>= 1) {
    const bool on = (wo & step) != 0;
#pragma unroll
    for (int j = 11; j >= 0; --j) y[j] = on ? (j >= step ? y[j - step] : 0u) : y[j];
  }
#pragma unroll
  for (int j = 0; j < 12; ++j) m[j] |= y[j];
}

// m |= byte ch at offset p (0 <= p < 48).
VS_HD void place_byte(uint32_t (&m)[12], uint32_t ch, int p) {
  const uint32_t v = ch << (8 * (p & 3));
#pragma unroll
  for (int j = 0; j < 12; ++j) m[j] |= (p >> 2) == j ? v : 0u;
}


VS_HD uint64_t position_seed(int64_t seed, int64_t position) {
  // magnitudes (also of INT64_MIN) and signs
  const uint64_t sa = seed < 0 ? 0 - static_cast<uint64_t>(seed) : static_cast<uint64_t>(seed);
  const uint64_t pa = position < 0 ? 0 - static_cast<uint64_t>(position) : static_cast<uint64_t>(position);
  const int s1 = seed < 0 ? 1 : 0, s2 = position < 0 ? 1 : 0;
  uint32_t t1[5], t2[5];
  const int n1 = decimal_text(sa, t1);
  const int n2 = decimal_text(pa, t2);
  uint32_t m[12];
#pragma unroll
  for (int j = 0; j < 12; ++j) m[j] = 0;
  place_byte(m, s1 ? '-' : 0u, 0);  // (a zero byte adds nothing)
  place(m, t1, s1);
  place_byte(m, ':', s1 + n1);
  place_byte(m, s2 ? '-' : 0u, s1 + n1 + 1);
  place(m, t2, s1 + n1 + 1 + s2);
  const int n = s1 + n1 + 1 + s2 + n2;  // (at most 41 bytes)
  uint64_t w[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) w[i] = (static_cast<uint64_t>(m[2 * i + 1]) << 32) | m[2 * i];
  return blake2b_8(w, n) & ((uint64_t(1) << 63) - 1);
}

VS_HD uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

VS_HD float position_uniform(int64_t seed, int64_t position) {
  return static_cast<float>(splitmix64(position_seed(seed, position)) >> 40) * 0x1p-24f;
}

#undef VS_HD

// The device form: one thread per (seed, position) pair.
__global__ __launch_bounds__(256) void k_uniforms(const int64_t* seeds, const int64_t* positions, int n, float* out) {
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i < n) out[i] = position_uniform(seeds[i], positions[i]);
}

// A speculative decode loop's per-sequence inputs ([4 + 2K + 1, n] int64, row-major: slot, last
// token, the token before it, that token's position (position - 2, with `position` the next
// token's), the K draft steps' positions (position - 1 + j), the target's K + 1 positions
// sequence-major (entry b (K + 1) + c of rows 4 + K ..: position - 1 + c)), advanced past one
// iteration whose verified tokens and counts (c tokens of sequence b emitted: position += c) are
// given, and the next iteration's 3K + 1 uniforms per sequence: draft draws [K, n] at -(4 (p + j)
// + 1), acceptances and residuals [n, K] at -(4 (p + j) + 2) and -(4 (p + j) + 3), the bonus [n]
// at -(4 (p + K) + 4), of the sequence's seed. Without counts the inputs stay and only the
// uniforms are computed. A group of G lanes (the power of two >= 3K + 1, so a group never
// straddles a wave) takes a sequence: every lane reads the position first, lane 0 then writes the
// new inputs (in the same wave: its stores follow the group's loads).
__global__ __launch_bounds__(256) void k_spec_advance(int64_t* inputs, int n, int K, int G, const int32_t* tokens,
                                                      const int32_t* counts, const int64_t* seeds, float* uniforms) {
  const int t = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  const int b = t / G, u = t % G;
  if (b >= n) return;  // (whole groups)
  const int64_t pos0 = inputs[3 * static_cast<int64_t>(n) + b] + 2;
  const int c = counts ? counts[b] : 0;
  const int64_t pos = pos0 + c;
  if (u < 3 * K + 1) {
    int64_t q;
    int64_t at;
    if (u < K) {
      q = -(4 * (pos + u) + 1);
      at = static_cast<int64_t>(u) * n + b;
    } else if (u < 2 * K) {
      q = -(4 * (pos + (u - K)) + 2);
      at = static_cast<int64_t>(K) * n + static_cast<int64_t>(b) * K + (u - K);
    } else if (u < 3 * K) {
      q = -(4 * (pos + (u - 2 * K)) + 3);
      at = 2 * static_cast<int64_t>(K) * n + static_cast<int64_t>(b) * K + (u - 2 * K);
    } else {
      q = -(4 * (pos + K) + 4);
      at = 3 * static_cast<int64_t>(K) * n + b;
    }
    uniforms[at] = position_uniform(seeds[b], q);
  }
  if (counts && u == 0) {
    const int32_t* tk = tokens + static_cast<int64_t>(b) * (K + 1);
    const int64_t last = inputs[static_cast<int64_t>(n) + b];
    inputs[static_cast<int64_t>(n) + b] = tk[c - 1];
    inputs[2 * static_cast<int64_t>(n) + b] = c >= 2 ? static_cast<int64_t>(tk[c - 2]) : last;
    inputs[3 * static_cast<int64_t>(n) + b] = pos - 2;
    for (int j = 0; j < K; ++j) inputs[static_cast<int64_t>(4 + j) * n + b] = pos - 1 + j;
    for (int j = 0; j <= K; ++j) inputs[static_cast<int64_t>(4 + K) * n + static_cast<int64_t>(b) * (K + 1) + j] = pos - 1 + j;
  }
}

}  // namespace vs_host
