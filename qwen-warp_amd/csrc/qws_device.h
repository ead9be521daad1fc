// qws device helpers: Philox4x32-10, order keys, the fixed-point weight definition, block reductions.
// Every floating-point expression here is compiled with -ffp-contract=off: each operation is one IEEE
// rounding, as in the CPU definition (oracle/sampler.py), so CPU and GPU agree bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qws.h"

namespace qws {

typedef unsigned __int128 u128;

constexpr int NT = 512;                  // threads per workgroup of both sampling kernels
constexpr int NWAVE = NT / 64;
constexpr int D_EXP = 38;                // weights below 2^-38 of the top exponent are dropped
constexpr int FB = 64;                   // fine bins per power of two (a = x / T in log2 units)
constexpr int NEXP = D_EXP + 1;          // exponents inside a weight window
constexpr int NBIN = NEXP * FB;          // fine bins inside a weight window (2496)
constexpr int CAP = 1024;                // elements a first-pass workgroup may hand to the resolver
constexpr int MAXIV = 3;                 // gathered bin intervals per first-pass workgroup
constexpr int MAXG = 128;                // chunks per row
constexpr double A_CLAMP = 1125899906842624.0;  // 2^50
constexpr double LOG2E = 1.4426950408889634;    // 0x1.71547652b82fep+0

// table word of the per-chunk processor state in LDS
constexpr uint32_t TB_CNT = 0xFFFFu;          // generated-token count (bits 0..15)
constexpr int TB_SLOT_SHIFT = 16;             // bias slot + 1 (bits 16..26)
constexpr uint32_t TB_SLOT = 0x7FFu;
constexpr uint32_t TB_STOP = 1u << 29;
constexpr uint32_t TB_PROMPT = 1u << 30;

// ---------------------------------------------------------------------------------------------- Philox4x32-10
// Random123's Philox4x32 with 10 rounds; the same round function as engine/src/mtp_sample.cu:10-23.
__host__ __device__ inline void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; r++) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}
// 24-bit uniform of counter (position, stream, row_key, 0), key = seed; word 0 = .x, 1 = .y
__host__ __device__ inline uint32_t draw_u24(uint64_t seed, uint32_t position, uint32_t stream, uint32_t row_key, int word) {
  uint32_t c[4] = {position, stream, row_key, 0u};
  philox(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  return c[word] >> 8;
}

// ---------------------------------------------------------------------------------------------- order
// Order-preserving key of an fp32 value, -0 folded into +0: larger key = earlier in rank order.
__device__ inline uint32_t okey(float x) {
  const uint32_t u = __float_as_uint(x + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float okey_val(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }
constexpr uint32_t KEY_NEGINF = 0x007FFFFFu;  // okey(-inf)
// composite rank: larger = earlier (value desc, index asc), as mkkey (engine/src/mtp_sample.cu:31-35)
__device__ inline uint64_t comp(uint32_t key, uint32_t idx) { return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx); }

// ---------------------------------------------------------------------------------------------- weights
// a = clamp((double)x * kappa, +-2^50), kappa = (double)(1.0f / T) * LOG2E
__device__ inline double log2u(float x, double kappa) {
  double a = (double)x * kappa;
  a = a < -A_CLAMP ? -A_CLAMP : a;
  a = a > A_CLAMP ? A_CLAMP : a;
  return a;
}
// 2^f on [0, 1]: Taylor coefficients ln2^k / k!, fp32, Horner
__device__ inline float exp2_frac(float f) {
  float p = __uint_as_float(0x33DA929Fu);
  p = p * f; p = p + __uint_as_float(0x35B16011u);
  p = p * f; p = p + __uint_as_float(0x377FE5FEu);
  p = p * f; p = p + __uint_as_float(0x39218489u);
  p = p * f; p = p + __uint_as_float(0x3AAEC3FFu);
  p = p * f; p = p + __uint_as_float(0x3C1D955Bu);
  p = p * f; p = p + __uint_as_float(0x3D635847u);
  p = p * f; p = p + __uint_as_float(0x3E75FDF0u);
  p = p * f; p = p + __uint_as_float(0x3F317218u);
  p = p * f;
  return p + 1.0f;
}
struct W {
  long long bin;  // floor(a * 64): absolute fine bin
  int n;          // floor(a)
  uint32_t mu;    // 24-bit mantissa of 2^(a - n)
};
__device__ inline W weigh(double a) {
  W w;
  const double fa = floor(a);
  w.bin = (long long)floor(a * 64.0);
  w.n = (int)fa;
  const float fr = (float)(a - fa);
  w.mu = (uint32_t)(exp2_frac(fr) * 8388608.0f);
  return w;
}
// weight in units of 2^(N - D_EXP - 23): mu << (n - N + D_EXP), 0 below the window
__device__ inline uint64_t wunits(const W& w, int N) {
  const int sh = w.n - N + D_EXP;
  return sh < 0 ? 0ull : ((uint64_t)w.mu << sh);
}

// ---------------------------------------------------------------------------------------------- block helpers
__device__ inline int lane_id() { return threadIdx.x & 63; }
__device__ inline int wave_id() { return threadIdx.x >> 6; }

template <typename T>
__device__ inline T wave_sum(T v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ inline u128 shfl_xor_u128(u128 v, int o) {
  const uint64_t lo = __shfl_xor((unsigned long)(uint64_t)v, o, 64);
  const uint64_t hi = __shfl_xor((unsigned long)(uint64_t)(v >> 64), o, 64);
  return ((u128)hi << 64) | lo;
}
__device__ inline u128 wave_sum_u128(u128 v) {
  for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u128(v, o);
  return v;
}
// Block-wide sum of a u128 (every thread gets the total).  red: LDS scratch of NWAVE u128.
__device__ inline u128 block_sum_u128(u128 v, u128* red) {
  v = wave_sum_u128(v);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  u128 t = 0;
  for (int i = 0; i < NWAVE; i++) t += red[i];
  return t;
}
// Block-wide inclusive prefix sum of a u128 in thread order; returns the inclusive prefix, *total = sum.
__device__ inline u128 block_scan_u128(u128 v, u128* red, u128* total) {
  const int lane = lane_id(), w = wave_id();
  u128 s = v;
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t lo = __shfl_up((unsigned long)(uint64_t)s, o, 64);
    const uint64_t hi = __shfl_up((unsigned long)(uint64_t)(s >> 64), o, 64);
    if (lane >= o) s += ((u128)hi << 64) | lo;
  }
  __syncthreads();
  if (lane == 63) red[w] = s;
  __syncthreads();
  u128 before = 0, t = 0;
  for (int i = 0; i < NWAVE; i++) {
    if (i < w) before += red[i];
    t += red[i];
  }
  *total = t;
  return before + s;
}

// max of (key, lowest idx) pairs packed as comp(); 0 = none
__device__ inline uint64_t wave_max_u64(uint64_t v) {
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = __shfl_xor((unsigned long)v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}
__device__ inline uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  v = wave_max_u64(v);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  uint64_t t = 0;
  for (int i = 0; i < NWAVE; i++) t = red[i] > t ? red[i] : t;
  return t;
}

}  // namespace qws
