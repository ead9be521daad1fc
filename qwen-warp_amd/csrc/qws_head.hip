// qws candidate select + exact rescore over the quantised head's approximate logits (the reference's
// smk_headq_select_rescore(_ids): engine/include/head_q.h:29-38; its definition, engine/src/head_q.cu:124-302).
//
// Input: approximate logits [T][N] fp32 (a quantised lm_head's output), the BF16 head w [rows][K] and the hidden
// states x [T][K] (bf16).  Output per row t: the R best candidates by approximate logit (larger value first, then the
// lower index; NaN never a candidate), their logits recomputed from the BF16 head (fp32 accumulation of exact bf16
// products) and written over the approximate values, and the argmax over those exact values (lowest token id on
// ties).  Four launches, stream-ordered and allocation-free (`ws` from the caller):
//   k_hs_tile     T x tiles x 256: a radix select (12-, 12- and 8-bit digits of the order key, LDS histograms) of
//                 each 4,096-logit tile's R best keys; ties at the tile's threshold key go to the lowest indices, in
//                 index order by block scans.  Every top-R key of a row is among the top R of its tile.
//   k_hs_row      T x 256: the same radix select over the row's tile winners (64-bit keys: value, then index, all
//                 distinct), then one wave sorts the R winners by a 64-lane bitonic network;
//   k_hs_rescore  T x ceil(R / 4) x 256: one wave per candidate, bf16 dot2 products accumulated in fp32;
//   k_hs_argmax   T x 64: the argmax over the exact candidate logits.
#include "qws_device.h"

namespace qws {

constexpr int HS_NT = 256;                       // threads of the select kernels
constexpr int HS_EPT = 16;                       // logits per thread of a tile (four float4 loads)
constexpr int HS_TILE = HS_NT * HS_EPT;          // 4,096 logits per tile
constexpr int HS_TILES = 64;                     // tiles per row at most: N <= 262,144
constexpr int HS_RMAX = 64;                      // candidates per row at most
constexpr int HS_ROWS = 16;                      // rows per call at most
constexpr int HS_LIST = HS_TILES * HS_RMAX;      // tile winners per row at most (4,096: 16 per thread of k_hs_row)

struct HsLayout {  // byte offsets in ws
  static constexpr size_t cand = 0;                                    // int [HS_ROWS][HS_RMAX] candidates by rank (-1: none)
  static constexpr size_t exact = cand + HS_ROWS * HS_RMAX * 4;        // float [HS_ROWS][HS_RMAX] their exact logits
  static constexpr size_t list = exact + HS_ROWS * HS_RMAX * 4;        // u64 [HS_ROWS][HS_TILES][HS_RMAX] tile winners (0: empty)
  static constexpr size_t total = list + (size_t)HS_ROWS * HS_LIST * 8;
};

// Order-preserving 32-bit key of a logit (-0 below +0, as the definition's ord32); NaN -> 0, below every other value
// (no other value maps to 0), so it is never a candidate.
__device__ inline uint32_t hs_ord(float f) {
  if (f != f) return 0u;
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One digit of a most-significant-first radix select over the block's keys: given the histogram `h` (256 bins, LDS)
// of the keys that match the digits chosen so far and `above` keys known to be larger, wave 0 finds the bin (from
// the top) where the running count reaches `need` and stores {bin, keys above that bin, keys in that bin} in
// sel[0..2]; sel[0] = -1 when fewer than `need` keys remain.  Called by the whole block; ends with a barrier.
__device__ inline void hs_pick_digit(const uint32_t* h, int above, int need, int* sel) {
  if (wave_id() == 0) {
    const int lane = lane_id();
    // lane l holds bins 255 - 4l .. 252 - 4l, the larger ones first
    uint32_t c[4];
#pragma unroll
    for (int i = 0; i < 4; i++) c[i] = h[255 - 4 * lane - i];
    const uint32_t mine = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_scan_incl<uint32_t>(mine);
    uint32_t run = (uint32_t)above + incl - mine;
    int bin = -1;
    uint32_t before = 0, inbin = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (bin < 0 && run + c[i] >= (uint32_t)need) {
        bin = 255 - 4 * lane - i;
        before = run;
        inbin = c[i];
      }
      run += c[i];
    }
    const int l = first_lane(bin >= 0);
    if (lane == (l < 64 ? l : 0)) {
      sel[0] = l < 64 ? bin : -1;
      sel[1] = (int)before;
      sel[2] = (int)inbin;
    }
  }
  bar();
}

// hs_pick_digit over a 4,096-bin histogram (a 12-bit digit): each thread sums 16 bins, wave 0 finds the 16-bin group
// where the running count reaches `need` (the 256 group sums as hs_pick_digit's bins), then the bin inside it.  part:
// 256 words of LDS.  Called by the whole block (HS_NT = 256 threads); ends with a barrier.
__device__ inline void hs_pick_digit12(const uint32_t* h, int above, int need, int* sel, uint32_t* part) {
  static_assert(HS_NT == 256, "a group of 16 bins per thread");
  const int tid = threadIdx.x;
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < 16; i++) c += h[4095 - 16 * tid - i];  // group tid: bins 4095 - 16 tid down to 4080 - 16 tid
  part[255 - tid] = c;  // as a 256-bin histogram: group tid is "bin" 255 - tid
  bar();
  hs_pick_digit(part, above, need, sel);
  const int q = sel[0];
  if (q >= 0 && wave_id() == 0) {  // uniform in the wave: the bin inside group 255 - q, from the top
    const int lane = lane_id(), grp = 255 - q;
    const uint32_t v = lane < 16 ? h[4095 - 16 * grp - lane] : 0u;
    const uint32_t incl = wave_scan_incl<uint32_t>(v) + (uint32_t)sel[1];
    const int i = first_lane(lane < 16 && incl >= (uint32_t)need);
    const uint32_t bin_before = readlane<uint32_t>(incl - v, i), bin_cnt = readlane<uint32_t>(v, i);
    if (lane == 0) {
      sel[0] = 4095 - 16 * grp - i;
      sel[1] = (int)bin_before;
      sel[2] = (int)bin_cnt;
    }
  }
  bar();
}

// Tile winners: the R best keys of tile `blockIdx.x` of row `blockIdx.y` (fewer when the tile holds fewer non-NaN
// logits) written to the row's list slot as composite keys (key << 32 | ~index), the rest of the slot 0.  The radix
// select takes a 12-bit digit, a 12-bit digit and an 8-bit digit: the first digit spreads the tile's keys over 4,096
// bins, so far fewer lanes of a wave add into one bin (an 8-bit first digit puts most logits of a row in a handful of
// bins: sign and high exponent bits).
__global__ void __launch_bounds__(HS_NT) k_hs_tile(const float* logits, int N, int R, unsigned long long* list) {
  __shared__ uint32_t s_h[2][4096];  // digit histograms, alternating (one is cleared while the other is read)
  __shared__ uint32_t s_part[256];
  __shared__ int s_sel[3], s_slot;
  __shared__ uint32_t s_red[HS_NT / 64];
  const int t = blockIdx.y, tile = blockIdx.x, tid = threadIdx.x;
  const int lo = tile * HS_TILE;
  const float* row = logits + (size_t)t * N;
  uint32_t k[HS_EPT];  // element 4s + j of this thread: index lo + s * 1024 + tid * 4 + j
#pragma unroll
  for (int s = 0; s < HS_EPT / 4; s++) {
    const int i0 = lo + s * (HS_NT * 4) + tid * 4;
    float4 v = make_float4(NAN, NAN, NAN, NAN);
    if (i0 < N) v = *(const float4*)(row + i0);  // N % 4 == 0: whole vectors
    k[4 * s] = hs_ord(v.x);
    k[4 * s + 1] = hs_ord(v.y);
    k[4 * s + 2] = hs_ord(v.z);
    k[4 * s + 3] = hs_ord(v.w);
  }
  // the R-th largest key theta (0 when the tile has at most R non-NaN keys: all of them are taken)
  uint32_t theta = 0u;
  int gt = 0;
  bool whole = false;  // theta ends a digit whose bin holds exactly the keys still needed: every key >= theta is taken
  for (int i = tid; i < 4096; i += HS_NT) s_h[0][i] = 0u;
  if (tid == 0) s_slot = 0;
  bar();
  for (int level = 0; level < 3; level++) {
    const int sh = level == 0 ? 20 : level == 1 ? 8 : 0, wd = level == 2 ? 8 : 12;  // digits: bits 31-20, 19-8, 7-0
    const uint32_t dmask = (1u << wd) - 1u;
    uint32_t* h = s_h[level & 1];
#pragma unroll
    for (int e = 0; e < HS_EPT; e++)
      if (k[e] && (level == 0 || (k[e] >> (sh + wd)) == (theta >> (sh + wd)))) atomicAdd(&h[(k[e] >> sh) & dmask], 1u);
    const int nnext = level == 0 ? 4096 : 256;  // the next digit's histogram
    for (int i = tid; i < nnext; i += HS_NT) s_h[(level & 1) ^ 1][i] = 0u;
    bar();
    if (wd == 12)
      hs_pick_digit12(h, gt, R, s_sel, s_part);
    else
      hs_pick_digit(h, gt, R, s_sel);
    const int d = s_sel[0];
    if (d < 0) {  // fewer than R keys (at level 0: fewer than R non-NaN logits in the tile)
      theta = 0u;
      gt = 0;
      break;
    }
    theta |= (uint32_t)d << sh;
    gt = s_sel[1];
    whole = gt + s_sel[2] == R && theta != 0u;  // uniform
    if (whole) break;
  }
  unsigned long long* slot = list + ((size_t)t * HS_TILES + tile) * HS_RMAX;
  if (whole) {  // the keys >= theta (the crossing bin's lowest key) are exactly R: no tie to break
#pragma unroll
    for (int e = 0; e < HS_EPT; e++) {
      if (k[e] >= theta) {
        const uint32_t idx = (uint32_t)(lo + (e >> 2) * (HS_NT * 4) + tid * 4 + (e & 3));
        slot[atomicAdd(&s_slot, 1)] = ((unsigned long long)k[e] << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
      }
    }
    bar();
    for (int i = s_slot + tid; i < HS_RMAX; i += HS_NT) slot[i] = 0ull;
    return;
  }
  // keys above theta, then the first R - gt keys equal to theta in index order (block scans over the four rounds)
  const int rem = theta ? R - gt : 0;
  int run = 0;
#pragma unroll
  for (int s = 0; s < HS_EPT / 4; s++) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) c += (theta && k[4 * s + j] == theta) ? 1 : 0;
    uint32_t tot;
    int ex = run + (int)block_scan_incl<HS_NT / 64, uint32_t>((uint32_t)c, s_red, &tot) - c;
    run += (int)tot;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t kk = k[4 * s + j];
      bool take = kk > theta;
      if (theta && kk == theta) take = ex++ < rem;
      if (take) {
        const uint32_t idx = (uint32_t)(lo + s * (HS_NT * 4) + tid * 4 + j);
        slot[atomicAdd(&s_slot, 1)] = ((unsigned long long)kk << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
      }
    }
  }
  bar();
  for (int i = s_slot + tid; i < HS_RMAX; i += HS_NT) slot[i] = 0ull;
}

// Row select: the R best of the row's tile winners (distinct 64-bit keys) by 12-, 12- and 8-bit digits of the value
// key, then of the index, then sorted by one wave; cand[t][r] = the row index of rank r (-1 past the winners).
__global__ void __launch_bounds__(HS_NT) k_hs_row(int tiles, int R, const unsigned long long* list, int* cand) {
  constexpr int PT = HS_LIST / HS_NT;
  __shared__ uint32_t s_h[2][4096];  // digit histograms, alternating
  __shared__ uint32_t s_part[256];
  __shared__ int s_sel[3], s_n;
  __shared__ unsigned long long s_win[HS_RMAX];
  const int t = blockIdx.x, tid = threadIdx.x, lane = lane_id();
  const int n = tiles * HS_RMAX;
  const unsigned long long* l = list + (size_t)t * HS_LIST;
  unsigned long long k[PT];
#pragma unroll
  for (int e = 0; e < PT; e++) {
    const int i = e * HS_NT + tid;
    k[e] = i < n ? l[i] : 0ull;
  }
  unsigned long long theta = 0ull;
  int gt = 0;
  for (int i = tid; i < 4096; i += HS_NT) s_h[0][i] = 0u;
  if (tid == 0) s_n = 0;
  bar();
  for (int level = 0; level < 6; level++) {
    // digits: value key bits 31-20, 19-8, 7-0, then the index word's, as bits 63-52, 51-40, 39-32, 31-20, 19-8, 7-0
    const int wd = (level % 3 == 2) ? 8 : 12, sh = (level < 3 ? 32 : 0) + (level % 3 == 0 ? 20 : level % 3 == 1 ? 8 : 0);
    const uint32_t dmask = (1u << wd) - 1u;
    uint32_t* h = s_h[level & 1];
#pragma unroll
    for (int e = 0; e < PT; e++)
      if (k[e] && (level == 0 || (k[e] >> (sh + wd)) == (theta >> (sh + wd)))) atomicAdd(&h[(uint32_t)(k[e] >> sh) & dmask], 1u);
    const int nnext = (level % 3 == 1) ? 256 : 4096;  // the next digit's histogram
    for (int i = tid; i < nnext; i += HS_NT) s_h[(level & 1) ^ 1][i] = 0u;
    bar();
    if (wd == 12)
      hs_pick_digit12(h, gt, R, s_sel, s_part);
    else
      hs_pick_digit(h, gt, R, s_sel);
    const int d = s_sel[0];
    if (d < 0) {  // fewer than R winners: all of them
      theta = 0ull;
      break;
    }
    theta |= (unsigned long long)d << sh;
    gt = s_sel[1];
    if (gt + s_sel[2] == R && theta != 0ull) break;  // uniform: the keys >= theta (the bin's lowest) are exactly the R best
  }
  // the keys are distinct: those >= theta are exactly the R best (or every nonzero key when theta = 0)
#pragma unroll
  for (int e = 0; e < PT; e++)
    if (k[e] && k[e] >= theta) s_win[atomicAdd(&s_n, 1)] = k[e];
  bar();
  if (wave_id() == 0) {
    unsigned long long v = lane < s_n ? s_win[lane] : 0ull;
    // bitonic network, descending: in stage (kk, j) the lane pair (i, i ^ j) orders its keys by the direction of
    // block kk (larger key to the lower lane when i & kk == 0)
    for (int kk = 2; kk <= 64; kk <<= 1) {
      for (int j = kk >> 1; j > 0; j >>= 1) {
        const uint32_t olo = (uint32_t)__shfl_xor((int)(uint32_t)v, j), ohi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), j);
        const unsigned long long o = ((unsigned long long)ohi << 32) | olo;
        const bool desc = (lane & kk) == 0, lower = (lane & j) == 0;
        v = (lower == desc) ? (v > o ? v : o) : (v < o ? v : o);
      }
    }
    if (lane < R) cand[t * HS_RMAX + lane] = v ? (int)(0xFFFFFFFFu - (uint32_t)v) : -1;
  }
}

typedef __attribute__((__vector_size__(2 * sizeof(short)))) short hs_bf2;

// exact logit of candidate r of row t: one wave, K / 8 uint4 pairs of bf16 (16-byte aligned rows)
__global__ void __launch_bounds__(256) k_hs_rescore(const uint4* w, const uint4* x, int N, int K, int R, float* logits, const int* cand,
                                                    float* exact, const int* ids) {
  const int t = blockIdx.y, lane = lane_id();
  const int r = blockIdx.x * 4 + wave_id();
  if (r >= R) return;
  const int row = cand[t * HS_RMAX + r];
  if (row < 0) return;
  const int id = ids ? ids[row] : row;
  const int KV = K / 8;
  const uint4* wr = w + (size_t)id * KV;
  const uint4* xr = x + (size_t)t * KV;
  float a = 0.0f;
  constexpr int U = 5;  // uint4 pairs of a lane in flight together (K = 5,120: two rounds); the same accumulation order
  for (int i0 = lane; i0 < KV; i0 += 64 * U) {
    uint4 wv[U], xv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + 64 * u;
      if (i < KV) {
        wv[u] = wr[i];
        xv[u] = xr[i];
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (i0 + 64 * u >= KV) break;
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hs_bf2, wv[u].x), __builtin_bit_cast(hs_bf2, xv[u].x), a, false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hs_bf2, wv[u].y), __builtin_bit_cast(hs_bf2, xv[u].y), a, false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hs_bf2, wv[u].z), __builtin_bit_cast(hs_bf2, xv[u].z), a, false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hs_bf2, wv[u].w), __builtin_bit_cast(hs_bf2, xv[u].w), a, false);
    }
  }
  const float v = wave_sum<float>(a);
  if (lane == 0) {
    exact[t * HS_RMAX + r] = v;
    logits[(size_t)t * N + row] = v;
  }
}

// argmax over the exact candidate logits of row t: the larger value, then the lower token id (no candidate: 0); the
// candidates become token ids when `ids` maps the rows
__global__ void __launch_bounds__(64) k_hs_argmax(int R, int* cand, const float* exact, const int* ids, int* out_tok, float* out_val) {
  const int t = blockIdx.x, lane = threadIdx.x;
  int ci = lane < R ? cand[t * HS_RMAX + lane] : -1;
  if (ci >= 0 && ids) ci = ids[ci];
  const float cv = ci >= 0 ? exact[t * HS_RMAX + lane] : 0.0f;
  const uint64_t key = ci >= 0 ? (((uint64_t)hs_ord(cv) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)ci)) : 0ull;
  const uint64_t m = wave_max_u64(key);
  const int wl = first_lane(m != 0ull && key == m);
  if (ids && lane < R) cand[t * HS_RMAX + lane] = ci;
  if (lane == 0) {
    out_tok[t] = wl < 64 ? (int)(0xFFFFFFFFu - (uint32_t)m) : 0;
    if (out_val) out_val[t] = wl < 64 ? exact[t * HS_RMAX + wl] : -INFINITY;
  }
}

}  // namespace qws

extern "C" size_t qws_head_ws_bytes(void) { return qws::HsLayout::total; }
extern "C" const int* qws_head_ws_cand(const void* ws) { return (const int*)((const char*)ws + qws::HsLayout::cand); }
extern "C" const float* qws_head_ws_exact(const void* ws) { return (const float*)((const char*)ws + qws::HsLayout::exact); }

extern "C" int qws_head_select_rescore(float* logits, const void* w_bf16, const void* x, int N, int K, int T, int R, int* out_tok, float* out_val, void* ws,
                                       void* stream, const int* ids) {
  using namespace qws;
  if (!logits || !w_bf16 || !x || !out_tok || !ws || ((uintptr_t)ws & 255) || ((uintptr_t)logits & 15) || ((uintptr_t)w_bf16 & 15) ||
      ((uintptr_t)x & 15))
    return QWS_ERR_INVALID;
  if (T < 1 || T > HS_ROWS || R < 1 || R > HS_RMAX || N < 4 || (N & 3) || K < 8 || (K & 7)) return QWS_ERR_INVALID;
  const int tiles = (N + HS_TILE - 1) / HS_TILE;
  if (tiles > HS_TILES) return QWS_ERR_NOT_SUPPORTED;
  char* b = (char*)ws;
  int* cand = (int*)(b + HsLayout::cand);
  float* exact = (float*)(b + HsLayout::exact);
  unsigned long long* list = (unsigned long long*)(b + HsLayout::list);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_hs_tile, dim3(tiles, T), dim3(HS_NT), 0, st, logits, N, R, list);
  hipLaunchKernelGGL(k_hs_row, dim3(T), dim3(HS_NT), 0, st, tiles, R, list, cand);
  hipLaunchKernelGGL(k_hs_rescore, dim3((R + 3) / 4, T), dim3(256), 0, st, (const uint4*)w_bf16, (const uint4*)x, N, K, R, logits, cand, exact, ids);
  hipLaunchKernelGGL(k_hs_argmax, dim3(T), dim3(64), 0, st, R, cand, exact, ids, out_tok, out_val);
  return (int)hipGetLastError();
}
