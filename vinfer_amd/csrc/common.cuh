// Shared device helpers for the sampler kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vs {

constexpr int kWave = 64;
constexpr int kThreads = 1024;  // one workgroup per row
constexpr int kWaves = kThreads / kWave;
constexpr int kBlk = 8;  // elements per block: one 16-byte bf16 load, two for fp32
constexpr int kMaxStripes = 64;  // V <= kMaxStripes * kThreads * kBlk = 524288
constexpr int kMassShift = 42;   // masses are fixed-point: q = rint(p~ * 2^42), p~ <= 1
constexpr double kMassScale = 4398046511104.0;  // 2^42

typedef unsigned long long u64;
typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ ushort2_t ones2() { return ushort2_t{1, 1}; }
// Ordered 16-bit keys (unsigned order = numeric order) of both bf16 values of a word at once:
// each half xor (sign ? 0xFFFF : 0x8000), the sign spread over its half by a packed arithmetic
// shift (v_pk_ashrrev_i16).
__device__ __forceinline__ uint32_t ok16x2(uint32_t w) {
  const short2_t sg = __builtin_bit_cast(short2_t, w) >> static_cast<short>(15);
  return w ^ (__builtin_bit_cast(uint32_t, sg) | 0x80008000u);
}

// ---- global pointers --------------------------------------------------------------------------
// Pointers that reach a kernel inside an argument struct are generic: loads through them compile
// to flat loads, which count against both the vector-memory and the LDS wait counters, so every
// LDS wait would also wait for the row loads in flight. Casting through the global address
// space lets the compiler emit global (and, for uniform addresses, scalar) loads instead.
template <class T>
__device__ __forceinline__ T* as_global(T* p) {
  return (T*)((__attribute__((address_space(1))) T*)p);
}

// A load through an explicitly global pointer (never a flat load).
template <class T>
__device__ __forceinline__ T ld_global(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}
// The same for 16 bytes (through a vector type: uint4's copy constructor takes no address space).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_global_u4(const uint4* p) {
  const u32x4_t v = ld_global(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- ordered keys ---------------------------------------------------------------------------
// A 32-bit key whose unsigned order is the numeric order of fp32 values, with -0.0 folded onto
// +0.0 (they compare equal) and every NaN mapped above +inf.
__device__ __forceinline__ uint32_t key_of(float x) {
  if (x != x) return 0xFFFFFFFFu;
  if (x == 0.0f) x = 0.0f;
  uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float val_of(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(b);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// ---- exp(d), d <= 0, in fp64 -------------------------------------------------------------------
// d = (16k + j) ln2/16 + r with |r| <= ln2/32, so exp(d) = 2^k (t_j + t_j (e^r - 1)) with
// t_j = 2^(j/16) (correctly rounded, below) and e^r - 1 from its Taylor series through r^7
// (the first omitted term is below 2e-18). The last fma rounds once; t_j's own rounding adds at
// most half an ulp. About 15 fp64 operations where the library exp takes about 35: the masses
// evaluate one per populated key and are bound by VALU issue.
constexpr double kExp2Sixteenths[16] = {
    0x1.0000000000000p+0, 0x1.0b5586cf9890fp+0, 0x1.172b83c7d517bp+0, 0x1.2387a6e756238p+0,
    0x1.306fe0a31b715p+0, 0x1.3dea64c123422p+0, 0x1.4bfdad5362a27p+0, 0x1.5ab07dd485429p+0,
    0x1.6a09e667f3bcdp+0, 0x1.7a11473eb0187p+0, 0x1.8ace5422aa0dbp+0, 0x1.9c49182a3f090p+0,
    0x1.ae89f995ad3adp+0, 0x1.c199bdd85529cp+0, 0x1.d5818dcfba487p+0, 0x1.ea4afa2a490dap+0};
constexpr double kSixteenOverLn2 = 0x1.71547652b82fep+4;
constexpr double kLn2Over16Hi = 0x1.62e42fefa0000p-5;  // 36 bits: k * hi is exact for |k| < 2^17
constexpr double kLn2Over16Lo = 0x1.cf79abc9e3b3ap-44;

// The table in LDS (a lane-indexed read); exp_table_init() fills it, before a barrier. Thread 0
// stores the 16 constants as immediates: a lane-indexed read of a constant array would be a
// global load at the kernel's start, which the next wait for any load waits for.
__shared__ double g_exp2_16[16];
__device__ __forceinline__ void exp_table_init() {
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) g_exp2_16[i] = kExp2Sixteenths[i];
  }
}

__device__ __forceinline__ double exp_nonpos(double d0) {
  // (branch-free, so that independent evaluations interleave: below the smallest subnormal,
  // and for -inf and NaN, the result is selected to 0 at the end)
  const bool tiny = !(d0 >= -745.5);
  const double d = tiny ? 0.0 : d0;
  const double kd = __builtin_rint(d * kSixteenOverLn2);
  double r = __builtin_fma(-kd, kLn2Over16Hi, d);
  r = __builtin_fma(-kd, kLn2Over16Lo, r);
  double q = __builtin_fma(r, 1.0 / 5040.0, 1.0 / 720.0);
  q = __builtin_fma(r, q, 1.0 / 120.0);
  q = __builtin_fma(r, q, 1.0 / 24.0);
  q = __builtin_fma(r, q, 1.0 / 6.0);
  q = __builtin_fma(r, q, 0.5);
  const double em1 = __builtin_fma(r * r, q, r);  // e^r - 1
  const int k = static_cast<int>(kd);
  const double t = g_exp2_16[k & 15];
  const double y = __builtin_ldexp(__builtin_fma(t, em1, t), k >> 4);
  return tiny ? 0.0 : y;
}

// ---- fixed-point mass of one value ------------------------------------------------------------
// p~ = exp(z - m) in fp64 with z = fl32(x / T) (IEEE division), m the row's max z.
__device__ __forceinline__ double ptilde(float x, float T, float mz) {
  const float z = T == 1.0f ? x : x / T;  // (x / 1 is x: skip the division)
  return exp_nonpos(static_cast<double>(z) - static_cast<double>(mz));
}

// q = rint(p * 2^42) for p in [0, 1]: adding 2^52 rounds to an integer (ties to even, as rint)
// and leaves it in the low mantissa bits.
__device__ __forceinline__ u64 mass_q(double p) {
  const double b = __builtin_fma(p, kMassScale, 4503599627370496.0);  // + 2^52
  return static_cast<u64>(__double_as_longlong(b)) - 0x4330000000000000ull;
}

// ---- barriers ---------------------------------------------------------------------------------
// A workgroup barrier that orders LDS only. __syncthreads() also releases global memory, which on
// gfx950 waits for every outstanding global load and store of the wave (vmcnt counts both); use
// this one wherever threads exchange data through LDS alone, so prefetches stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- lanes of one wave exchanging LDS words without a workgroup barrier -------------------------
// A wave's LDS operations complete in program order, so lanes can pass words to each other
// through LDS with no barrier; but to the compiler the lanes are separate threads, and it may
// forward a lane's own earlier store to a later read of the same word (on a path where the lane
// did no atomic there itself) or move reads across the other lanes' updates. wave_lds_sync()
// keeps LDS reads and writes from moving or being forwarded across it (a wavefront-scope fence:
// no instruction); lds_peek() / lds_poke() read and write a word as relaxed atomics, which are
// never forwarded.
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }
template <class T>
__device__ __forceinline__ T lds_peek(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
template <class T>
__device__ __forceinline__ void lds_poke(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

// ---- uniform values ----------------------------------------------------------------------------
// A value every lane holds the same copy of (read from LDS, say), moved to a scalar register:
// branches on it are scalar branches and arithmetic with it takes a scalar operand.
__device__ __forceinline__ float uniform_f(float x) {
  return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(x)));
}
__device__ __forceinline__ uint32_t uniform_u(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int uniform_i(int x) { return __builtin_amdgcn_readfirstlane(x); }

// ---- wave primitives --------------------------------------------------------------------------
// Cross-lane steps use DPP (data-parallel primitives: a VALU operand read from another lane of
// the same 16-lane row, or broadcast across rows) rather than ds_bpermute shuffles, which go
// through the LDS crossbar and cost a round trip each.
__device__ __forceinline__ int lane_id() { return __lane_id(); }

namespace dpp {
constexpr int kXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kShr1 = 0x111;        // row_shr:1 (+ n - 1 for row_shr:n)
constexpr int kMirror = 0x140;      // row_mirror: lane 15 - i of the row
constexpr int kHalfMirror = 0x141;  // row_half_mirror: lane 7 - i of the half-row
constexpr int kBcast15 = 0x142;     // lane 15 of each row into the next row (row_mask picks rows)
constexpr int kBcast31 = 0x143;     // lane 31 into rows 2 and 3

// Lane-moved copy of x; lanes the control leaves without a source (or rows outside row_mask)
// read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t mov(uint32_t x) {
  if constexpr (ROW_MASK == 0xF && (CTRL < 0x100 || CTRL == kMirror || CTRL == kHalfMirror)) {
    // every lane has a source lane: no old value to keep
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), CTRL, 0xF, 0xF, false));
  }
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROW_MASK, 0xF, true));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ u64 mov(u64 x) {
  const uint32_t lo = mov<CTRL, ROW_MASK>(static_cast<uint32_t>(x));
  const uint32_t hi = mov<CTRL, ROW_MASK>(static_cast<uint32_t>(x >> 32));
  return (static_cast<u64>(hi) << 32) | lo;
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double mov(double x) {
  return __longlong_as_double(static_cast<long long>(mov<CTRL, ROW_MASK>(static_cast<u64>(__double_as_longlong(x)))));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int mov(int x) {
  return static_cast<int>(mov<CTRL, ROW_MASK>(static_cast<uint32_t>(x)));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float mov(float x) {
  return __uint_as_float(mov<CTRL, ROW_MASK>(__float_as_uint(x)));
}

// Lane 63's value, in every lane.
__device__ __forceinline__ uint32_t last(uint32_t x) { return __builtin_amdgcn_readlane(x, 63); }
__device__ __forceinline__ int last(int x) { return __builtin_amdgcn_readlane(x, 63); }
__device__ __forceinline__ u64 last(u64 x) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(x), 63);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(x >> 32), 63);
  return (static_cast<u64>(hi) << 32) | lo;
}
__device__ __forceinline__ double last(double x) {
  return __longlong_as_double(static_cast<long long>(last(static_cast<u64>(__double_as_longlong(x)))));
}
__device__ __forceinline__ float last(float x) { return __uint_as_float(last(__float_as_uint(x))); }

// Reduction with an associative, commutative op: every 16-lane row ends with its row total in
// all lanes, then rows 1 and 3 fold in rows 0 and 2, then row 3 folds in rows 0 + 1.
template <class T, class Op>
__device__ __forceinline__ T reduce(T v, Op op) {
  v = op(v, mov<kXor1>(v));
  v = op(v, mov<kXor2>(v));
  v = op(v, mov<kHalfMirror>(v));
  v = op(v, mov<kMirror>(v));
  v = op(v, mov<kBcast15, 0xA>(v));
  v = op(v, mov<kBcast31, 0xC>(v));
  return last(v);
}
}  // namespace dpp

// Sum over the wave's 64 lanes, in every lane (32/64-bit integers).
template <class T>
__device__ __forceinline__ T wave_sum(T v) {
  return dpp::reduce(v, [](T a, T b) { return a + b; });
}

__device__ __forceinline__ u64 wave_max_u64(u64 v) {
  return dpp::reduce(v, [](u64 a, u64 b) { return a > b ? a : b; });
}

// Inclusive prefix sum over the wave's lanes (32/64-bit integers): Hillis-Steele steps of 1, 2,
// 4 and 8 lanes inside each 16-lane row, then the row carries.
template <class T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  v += dpp::mov<dpp::kShr1>(v);
  v += dpp::mov<dpp::kShr1 + 1>(v);
  v += dpp::mov<dpp::kShr1 + 3>(v);
  v += dpp::mov<dpp::kShr1 + 7>(v);
  v += dpp::mov<dpp::kBcast15, 0xA>(v);
  v += dpp::mov<dpp::kBcast31, 0xC>(v);
  return v;
}

// Set bits of a wave mask in the lanes below this one (v_mbcnt: two instructions).
__device__ __forceinline__ uint32_t lanes_below(u64 m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

// A 64-bit value of one lane, in every lane.
__device__ __forceinline__ u64 readlane64(u64 x, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(x), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(x >> 32), lane);
  return (static_cast<u64>(hi) << 32) | lo;
}

// Inclusive scan within each row of 16 lanes.
template <class T>
__device__ __forceinline__ T row_incl_scan(T v) {
  v += dpp::mov<dpp::kShr1>(v);
  v += dpp::mov<dpp::kShr1 + 1>(v);
  v += dpp::mov<dpp::kShr1 + 3>(v);
  v += dpp::mov<dpp::kShr1 + 7>(v);
  return v;
}

// Inclusive scan within each half of the wave (lanes 0-31, 32-63): lane 31 holds the sum of the
// first half, lane 63 of the second.
template <class T>
__device__ __forceinline__ T half_incl_scan(T v) {
  v += dpp::mov<dpp::kShr1>(v);
  v += dpp::mov<dpp::kShr1 + 1>(v);
  v += dpp::mov<dpp::kShr1 + 3>(v);
  v += dpp::mov<dpp::kShr1 + 7>(v);
  v += dpp::mov<dpp::kBcast15, 0xA>(v);
  return v;
}

// For every lane with `valid`, acc[key] op= v through `at(key, value)`, lanes sharing a key
// combined first: one LDS atomic per distinct key in the wave instead of one per lane (keys
// that many lanes share would otherwise serialise). All 64 lanes must be active.
template <class T, class Op, class At>
__device__ __forceinline__ void wave_grouped(uint32_t key, T v, bool valid, Op op, At at) {
  u64 act = __ballot(valid);
  while (act) {
    const int leader = __ffsll(static_cast<long long>(act)) - 1;
    const uint32_t k0 = __builtin_amdgcn_readlane(key, leader);
    const bool mine = valid && key == k0;
    const u64 same = __ballot(mine);
    const T s = dpp::reduce(mine ? v : T(0), op);
    if (lane_id() == leader) at(k0, s);
    act &= ~same;
  }
}

// ---- workgroup primitives (kThreads threads, all must call) ------------------------------------
// `red` must hold kWaves entries of T.
template <class T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  lds_barrier();
  if (lane_id() == 0) red[w] = v;
  lds_barrier();
  T s = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) s += red[i];
  return s;
}

__device__ __forceinline__ u64 block_max_u64(u64 v, u64* red) {
  v = wave_max_u64(v);
  const int w = threadIdx.x / kWave;
  lds_barrier();
  if (lane_id() == 0) red[w] = v;
  lds_barrier();
  u64 s = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) s = red[i] > s ? red[i] : s;
  return s;
}

// A workgroup sum and max at once (one pair of barriers). `red` must hold 2 * kWaves entries.
__device__ __forceinline__ void block_sum_max_u64(u64 sv, u64 mv, u64* red, u64* sum, u64* mx) {
  sv = wave_sum(sv);
  mv = wave_max_u64(mv);
  const int w = threadIdx.x / kWave;
  lds_barrier();
  if (lane_id() == 0) {
    red[w] = sv;
    red[kWaves + w] = mv;
  }
  lds_barrier();
  u64 s = 0, m = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    s += red[i];
    m = red[kWaves + i] > m ? red[kWaves + i] : m;
  }
  *sum = s;
  *mx = m;
}

// Exclusive prefix sum over the workgroup in thread order; returns the total in *total.
template <class T>
__device__ __forceinline__ T block_excl_scan(T v, T* red, T* total) {
  T inc = wave_incl_scan(v);
  const int w = threadIdx.x / kWave;
  lds_barrier();
  if (lane_id() == kWave - 1) red[w] = inc;
  lds_barrier();
  T base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    base += (i < w) ? red[i] : T(0);
    tot += red[i];
  }
  *total = tot;
  return base + inc - v;
}

}  // namespace vs
