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
constexpr int MAXIV = 2;                 // handed-over bin intervals per chunk: the top set and a window
constexpr int MAXG = 64;                 // chunks per row (V <= 64 * 4,096)
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
// a = clamp(x * kappa, +-2^22) in log2 units, kappa = (float)((double)(1.0f / T) * LOG2E).
// q = floor(a * 256): n = q >> 8 = floor(a), fine bin = q >> 2 = floor(a * 64);
// mu = (uint32)(TAB[q & 255] * (1 + r * (C1 + r * C2)) * 2^23), r = a * 256 - floor(a * 256).
constexpr float A_CLAMPF = 4194304.0f;  // 2^22
__device__ __constant__ uint32_t EXP2_TAB[256] = {
    0x3f800000, 0x3f8058d8, 0x3f80b1ed, 0x3f810b41, 0x3f8164d2, 0x3f81bea1, 0x3f8218af, 0x3f8272fc,
    0x3f82cd87, 0x3f832850, 0x3f838359, 0x3f83dea1, 0x3f843a29, 0x3f8495f0, 0x3f84f1f6, 0x3f854e3d,
    0x3f85aac3, 0x3f86078a, 0x3f866491, 0x3f86c1d9, 0x3f871f62, 0x3f877d2b, 0x3f87db35, 0x3f883981,
    0x3f88980f, 0x3f88f6dd, 0x3f8955ee, 0x3f89b541, 0x3f8a14d5, 0x3f8a74ad, 0x3f8ad4c6, 0x3f8b3523,
    0x3f8b95c2, 0x3f8bf6a4, 0x3f8c57ca, 0x3f8cb933, 0x3f8d1adf, 0x3f8d7cd0, 0x3f8ddf04, 0x3f8e417d,
    0x3f8ea43a, 0x3f8f073b, 0x3f8f6a81, 0x3f8fce0c, 0x3f9031dc, 0x3f9095f2, 0x3f90fa4d, 0x3f915eed,
    0x3f91c3d3, 0x3f922900, 0x3f928e72, 0x3f92f42c, 0x3f935a2b, 0x3f93c072, 0x3f9426ff, 0x3f948dd4,
    0x3f94f4f0, 0x3f955c53, 0x3f95c3ff, 0x3f962bf2, 0x3f96942d, 0x3f96fcb1, 0x3f97657d, 0x3f97ce92,
    0x3f9837f0, 0x3f98a197, 0x3f990b88, 0x3f9975c2, 0x3f99e046, 0x3f9a4b13, 0x3f9ab62b, 0x3f9b218d,
    0x3f9b8d3a, 0x3f9bf931, 0x3f9c6573, 0x3f9cd201, 0x3f9d3eda, 0x3f9dabfe, 0x3f9e196e, 0x3f9e872a,
    0x3f9ef532, 0x3f9f6387, 0x3f9fd228, 0x3fa04116, 0x3fa0b051, 0x3fa11fd9, 0x3fa18faf, 0x3fa1ffd2,
    0x3fa27043, 0x3fa2e102, 0x3fa3520f, 0x3fa3c36b, 0x3fa43516, 0x3fa4a70f, 0x3fa51958, 0x3fa58bef,
    0x3fa5fed7, 0x3fa6720e, 0x3fa6e595, 0x3fa7596c, 0x3fa7cd94, 0x3fa8420c, 0x3fa8b6d5, 0x3fa92bef,
    0x3fa9a15b, 0x3faa1718, 0x3faa8d26, 0x3fab0387, 0x3fab7a3a, 0x3fabf13f, 0x3fac6897, 0x3face041,
    0x3fad583f, 0x3fadd090, 0x3fae4934, 0x3faec22d, 0x3faf3b79, 0x3fafb519, 0x3fb02f0e, 0x3fb0a957,
    0x3fb123f6, 0x3fb19ee9, 0x3fb21a32, 0x3fb295d0, 0x3fb311c4, 0x3fb38e0e, 0x3fb40aaf, 0x3fb487a6,
    0x3fb504f3, 0x3fb58298, 0x3fb60094, 0x3fb67ee7, 0x3fb6fd92, 0x3fb77c95, 0x3fb7fbf0, 0x3fb87ba3,
    0x3fb8fbaf, 0x3fb97c14, 0x3fb9fcd2, 0x3fba7dea, 0x3fbaff5b, 0x3fbb8126, 0x3fbc034a, 0x3fbc85ca,
    0x3fbd08a4, 0x3fbd8bd8, 0x3fbe0f68, 0x3fbe9353, 0x3fbf179a, 0x3fbf9c3c, 0x3fc0213b, 0x3fc0a695,
    0x3fc12c4d, 0x3fc1b261, 0x3fc238d2, 0x3fc2bfa1, 0x3fc346cd, 0x3fc3ce57, 0x3fc4563f, 0x3fc4de85,
    0x3fc5672a, 0x3fc5f02e, 0x3fc67991, 0x3fc70353, 0x3fc78d75, 0x3fc817f7, 0x3fc8a2d8, 0x3fc92e1b,
    0x3fc9b9be, 0x3fca45c1, 0x3fcad226, 0x3fcb5eed, 0x3fcbec15, 0x3fcc799f, 0x3fcd078c, 0x3fcd95da,
    0x3fce248c, 0x3fceb3a1, 0x3fcf4319, 0x3fcfd2f4, 0x3fd06334, 0x3fd0f3d7, 0x3fd184df, 0x3fd2164c,
    0x3fd2a81e, 0x3fd33a54, 0x3fd3ccf1, 0x3fd45ff3, 0x3fd4f35b, 0x3fd58729, 0x3fd61b5e, 0x3fd6affa,
    0x3fd744fd, 0x3fd7da67, 0x3fd87039, 0x3fd90673, 0x3fd99d16, 0x3fda3421, 0x3fdacb94, 0x3fdb6371,
    0x3fdbfbb8, 0x3fdc9468, 0x3fdd2d82, 0x3fddc706, 0x3fde60f5, 0x3fdefb4e, 0x3fdf9613, 0x3fe03143,
    0x3fe0ccdf, 0x3fe168e7, 0x3fe2055b, 0x3fe2a23c, 0x3fe33f89, 0x3fe3dd44, 0x3fe47b6d, 0x3fe51a03,
    0x3fe5b907, 0x3fe65879, 0x3fe6f85b, 0x3fe798ab, 0x3fe8396a, 0x3fe8da99, 0x3fe97c38, 0x3fea1e47,
    0x3feac0c7, 0x3feb63b7, 0x3fec0719, 0x3fecaaec, 0x3fed4f30, 0x3fedf3e7, 0x3fee9910, 0x3fef3eab,
    0x3fefe4ba, 0x3ff08b3b, 0x3ff13231, 0x3ff1d99a, 0x3ff28177, 0x3ff329c9, 0x3ff3d290, 0x3ff47bcc,
    0x3ff5257d, 0x3ff5cfa4, 0x3ff67a41, 0x3ff72555, 0x3ff7d0df, 0x3ff87ce1, 0x3ff9295a, 0x3ff9d64a,
    0x3ffa83b3, 0x3ffb3194, 0x3ffbdfed, 0x3ffc8ec0, 0x3ffd3e0c, 0x3ffdedd2, 0x3ffe9e11, 0x3fff4ecb,
};
constexpr uint32_t EXP2_C1 = 0x3B317218u;  // fp32(ln2 / 256)
constexpr uint32_t EXP2_C2 = 0x3675FDF0u;  // fp32((ln2 / 256)^2 / 2)

__device__ inline float kappa_f(float temperature) { return (float)((double)(1.0f / temperature) * LOG2E); }
__device__ inline float log2u(float x, float kappa) {
  const float a = x * kappa;
  return fminf(fmaxf(a, -A_CLAMPF), A_CLAMPF);
}
struct W {
  int q;          // floor(a * 256)
  uint32_t mu;    // 24-bit mantissa of 2^(a - floor(a))
  __device__ inline int bin() const { return q >> 2; }
  __device__ inline int n() const { return q >> 8; }
};
// tab: the 256-entry table (LDS copy or EXP2_TAB)
__device__ inline W weigh(float a, const float* tab) {
  W w;
  const float t = a * 256.0f;
  const float fl = floorf(t);
  w.q = (int)fl;
  const float r = t - fl;
  float p = r * __uint_as_float(EXP2_C2);
  p = p + __uint_as_float(EXP2_C1);
  p = p * r;
  p = p + 1.0f;
  const float m = tab[w.q & 255] * p;
  w.mu = (uint32_t)(m * 8388608.0f);
  return w;
}
__device__ inline W weigh_c(float a) { return weigh(a, (const float*)EXP2_TAB); }
// weight in units of 2^(N - D_EXP - 23): mu << (n - N + D_EXP), 0 below the window
__device__ inline uint64_t wunits(const W& w, int N) {
  const int sh = w.n() - N + D_EXP;
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
