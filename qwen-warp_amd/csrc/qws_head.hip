// qws candidate select + exact rescore over the quantised head's approximate logits (the reference's
// smk_headq_select_rescore, engine/src/head_q.cu:124-302, engine/include/head_q.h:29-38).
//
// Input: approximate logits [T][N] fp32 (a quantised lm_head's output), the BF16 head w [N][K] and the hidden
// states x [T][K] (bf16).  Output per row t: the R best candidates by approximate logit (larger value first, then
// the lower index; NaN never a candidate), their logits recomputed from the BF16 head (fp32 accumulation of exact
// bf16 products) and written over the approximate values, and the argmax over those exact values (lowest index on
// ties).  Five launches, all stream-ordered and allocation-free (`ws` from the caller):
//   k_hq_chunkmax  T x NCH x 256: the best key of every 2,048-logit chunk (so that a row has more chunks than R);
//   k_hq_extract   T x NCH x 256: thr = the R-th largest chunk best of the row (R distinct keys are >= thr, so every
//                  top-R key is >= thr); a chunk whose best is >= thr lists its keys >= thr, at most its own R best
//                  (a top-R key of the row is among the top R of its chunk), so a row's list holds <= NCH * R keys;
//   k_hq_rank      T x 512: the R best of the row's list by exact rank (counting below 2,048 listed keys, an LDS
//                  bitonic sort above);
//   k_hq_rescore   T x ceil(R / 4) x 256: one wave per candidate, bf16 dot2 products accumulated in fp32;
//   k_hq_argmax    T x 64: the argmax over the exact candidate logits.
#include "qws_device.h"

namespace qws {

constexpr int HQ_CHUNK = 2048;                   // logits per chunk (256 threads x 8)
constexpr int HQ_NCH = 128;                      // chunks per row at most: N <= 262,144
constexpr int HQ_RMAX = 64;                      // candidates per row at most
constexpr int HQ_ROWS = 16;                      // rows per call at most
constexpr int HQ_LIST = HQ_NCH * HQ_RMAX;        // listed keys per row at most
constexpr int HQ_FLAT = 512;                     // chunk survivors ranked by counting at most (more: bitonic sort)

struct HqLayout {  // byte offsets in ws
  static constexpr size_t cnt = 0;                                   // int [HQ_ROWS] listed keys per row
  static constexpr size_t cm = 256;                                  // u32 [HQ_ROWS][HQ_NCH] chunk bests
  static constexpr size_t cand = cm + HQ_ROWS * HQ_NCH * 4;          // int [HQ_ROWS][HQ_RMAX] candidate ids by rank (-1: none)
  static constexpr size_t exact = cand + HQ_ROWS * HQ_RMAX * 4;      // float [HQ_ROWS][HQ_RMAX] their exact logits
  static constexpr size_t list = exact + HQ_ROWS * HQ_RMAX * 4;      // u64 [HQ_ROWS][HQ_LIST] listed keys
  static constexpr size_t total = list + (size_t)HQ_ROWS * HQ_LIST * 8;
};

// order-preserving 32-bit key of a logit; NaN -> 0 (never a candidate: every other value maps above 0)
__device__ inline uint32_t hq_ord(float f) {
  if (f != f) return 0u;
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline uint64_t hq_key(uint32_t o, uint32_t idx) { return ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - idx); }
__device__ inline uint32_t hq_idx(uint64_t k) { return 0xFFFFFFFFu - (uint32_t)k; }

__global__ void __launch_bounds__(256) k_hq_chunkmax(const float* lg, int N, uint32_t* cm, int* cnt) {
  const int t = blockIdx.y, c = blockIdx.x, tid = threadIdx.x;
  __shared__ uint32_t s_red[4];
  const float* row = lg + (size_t)t * N;
  uint32_t best = 0u;
#pragma unroll
  for (int i = 0; i < HQ_CHUNK / 1024; i++) {
    const int idx = c * HQ_CHUNK + (i * 256 + tid) * 4;
    if (idx < N) {  // N % 4 == 0
      const float4 v = *(const float4*)(row + idx);
      best = max(best, max(max(hq_ord(v.x), hq_ord(v.y)), max(hq_ord(v.z), hq_ord(v.w))));
    }
  }
  best = wave_max_u32(best);
  if (lane_id() == 0) s_red[wave_id()] = best;
  bar();
  if (tid == 0) {
    cm[t * HQ_NCH + c] = max(max(s_red[0], s_red[1]), max(s_red[2], s_red[3]));
    if (c == 0) cnt[t] = 0;
  }
}

// LDS bitonic sort of n2 (a power of two) keys, descending; every thread of the workgroup calls it
template <int NT>
__device__ void hq_sort_desc(uint64_t* k, int n2) {
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < n2 / 2; i += NT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = k[lo], b = k[hi];
        if (desc ? a < b : a > b) {
          k[lo] = b;
          k[hi] = a;
        }
      }
      bar();
    }
  }
}

__global__ void __launch_bounds__(256) k_hq_extract(const float* lg, int N, int R, const uint32_t* cm_all, int* cnt, uint64_t* list) {
  __shared__ uint32_t s_cm[HQ_NCH];
  __shared__ uint32_t s_thr;
  __shared__ int s_ns;
  __shared__ uint64_t s_k[HQ_CHUNK];
  const int t = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, nch = gridDim.x;
  if (tid < nch) s_cm[tid] = cm_all[t * HQ_NCH + tid];
  if (tid == 0) {
    s_thr = nch <= R ? 1u : 0xFFFFFFFFu;  // every non-NaN key when the chunks cannot hold R candidates each
    s_ns = 0;
  }
  bar();
  if (nch > R && tid < nch) {  // the R-th largest chunk best: its rank among the chunk bests is < R
    int above = 0;
    for (int j = 0; j < nch; j++) above += s_cm[j] > s_cm[tid] ? 1 : 0;
    if (above < R) atomicMin(&s_thr, s_cm[tid]);
  }
  bar();
  const uint32_t thr = max(s_thr, 1u);
  if (s_cm[c] < thr) return;  // uniform
  const float* row = lg + (size_t)t * N;
  uint64_t key[HQ_CHUNK / 256];
  int mine = 0;
#pragma unroll
  for (int i = 0; i < HQ_CHUNK / 1024; i++) {
    const int idx = c * HQ_CHUNK + (i * 256 + tid) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (idx < N) v = *(const float4*)(row + idx);
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t o = hq_ord(vv[j]);
      const bool in = idx < N && o >= thr;
      key[i * 4 + j] = in ? hq_key(o, (uint32_t)(idx + j)) : 0ull;
      mine += in ? 1 : 0;
    }
  }
  // the chunk's survivors into LDS (one slot atomic per wave)
  int slot;
  {
    const int inc = wave_scan_incl<int>(mine);
    int wb = 0;
    if (lane_id() == 63 && inc) wb = atomicAdd(&s_ns, inc);
    slot = readlane<int>(wb, 63) + inc - mine;
  }
#pragma unroll
  for (int i = 0; i < HQ_CHUNK / 256; i++)
    if (key[i]) s_k[slot++] = key[i];
  bar();
  const int ns = s_ns;
  uint64_t* out = list + (size_t)t * HQ_LIST;
  if (ns <= R) {
    if (tid == 0 && ns) {
      const int base = atomicAdd(&cnt[t], ns);
      for (int e = 0; e < ns; e++) out[base + e] = s_k[e];
    }
    return;
  }
  if (ns <= HQ_FLAT) {  // keys are distinct: a key is among the chunk's R best iff fewer than R keys are larger
    __shared__ int s_base;
    if (tid == 0) s_base = atomicAdd(&cnt[t], R);
    bar();
    for (int e = tid; e < ns; e += 256) {
      const uint64_t k = s_k[e];
      int rank = 0;
      for (int j = 0; j < ns; j++) rank += s_k[j] > k ? 1 : 0;
      if (rank < R) out[s_base + rank] = k;
    }
    return;
  }
  int n2 = 1;
  while (n2 < ns) n2 <<= 1;
  for (int e = ns + tid; e < n2; e += 256) s_k[e] = 0ull;
  bar();
  hq_sort_desc<256>(s_k, n2);
  if (tid == 0) {
    const int base = atomicAdd(&cnt[t], R);
    for (int e = 0; e < R; e++) out[base + e] = s_k[e];
  }
}

// The R best of a row's listed keys (distinct) -> cand[t][rank] (token ids), -1 past them.
__global__ void __launch_bounds__(512) k_hq_rank(int R, const int* cnt, const uint64_t* list, int* cand) {
  __shared__ uint64_t s_k[HQ_LIST];
  const int t = blockIdx.x, tid = threadIdx.x;
  const int n = min(cnt[t], HQ_LIST);
  const uint64_t* in = list + (size_t)t * HQ_LIST;
  for (int i = tid; i < n; i += 512) s_k[i] = in[i];
  for (int e = n + tid; e < R; e += 512) cand[t * HQ_RMAX + e] = -1;  // ranks no key takes (each slot written once)
  bar();
  if (n <= 2048) {
    for (int e = tid; e < n; e += 512) {
      const uint64_t k = s_k[e];
      int rank = 0;
      for (int j = 0; j < n; j++) rank += s_k[j] > k ? 1 : 0;
      if (rank < R) cand[t * HQ_RMAX + rank] = (int)hq_idx(k);
    }
    return;
  }
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (int e = n + tid; e < n2; e += 512) s_k[e] = 0ull;
  bar();
  hq_sort_desc<512>(s_k, n2);
  if (tid < R && tid < n) cand[t * HQ_RMAX + tid] = (int)hq_idx(s_k[tid]);
}

typedef __bf16 hq_bf2 __attribute__((ext_vector_type(2)));

// Exact logit of candidate (t, r): one wave, lane l takes the 16-byte column groups l, l + 64, ... of w[id] and
// x[t] (8 bf16 each), accumulated in fp32 by bf16 dot2 products, then a wave sum.
__global__ void __launch_bounds__(256) k_hq_rescore(const uint4* w, const uint4* x, int N, int K, int R, float* logits, const int* cand,
                                                     float* exact, const int* ids) {
  const int t = blockIdx.y, lane = lane_id();
  const int r = blockIdx.x * 4 + wave_id();
  if (r >= R) return;
  const int row = cand[t * HQ_RMAX + r];
  if (row < 0) return;
  const int id = ids ? ids[row] : row;
  const int KV = K / 8;
  const uint4* wr = w + (size_t)id * KV;
  const uint4* xr = x + (size_t)t * KV;
  float a = 0.0f;
  for (int i = lane; i < KV; i += 64) {
    const uint4 wv = wr[i], xv = xr[i];
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hq_bf2, wv.x), __builtin_bit_cast(hq_bf2, xv.x), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hq_bf2, wv.y), __builtin_bit_cast(hq_bf2, xv.y), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hq_bf2, wv.z), __builtin_bit_cast(hq_bf2, xv.z), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(hq_bf2, wv.w), __builtin_bit_cast(hq_bf2, xv.w), a, false);
  }
  const float v = wave_sum<float>(a);
  if (lane == 0) {
    exact[t * HQ_RMAX + r] = v;
    logits[(size_t)t * N + row] = v;
  }
}

// argmax over the exact candidate logits of row t: the larger value, then the lower token id (no candidate: 0)
__global__ void __launch_bounds__(64) k_hq_argmax(int R, int* cand, const float* exact, const int* ids, int* out_tok, float* out_val) {
  const int t = blockIdx.x, lane = threadIdx.x;
  int ci = lane < R ? cand[t * HQ_RMAX + lane] : -1;
  if (ci >= 0 && ids) ci = ids[ci];
  const float cv = ci >= 0 ? exact[t * HQ_RMAX + lane] : -INFINITY;
  // key: ordered value, then the lower id
  const uint64_t k = ci >= 0 ? (((uint64_t)hq_ord(cv) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)ci)) : 0ull;
  uint64_t m = k;
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) {
    const uint64_t o = __shfl_xor(m, sh);
    m = o > m ? o : m;
  }
  if (ids && lane < R) cand[t * HQ_RMAX + lane] = ci;  // candidates as token ids
  if (lane == 0) {
    out_tok[t] = m ? (int)(0xFFFFFFFFu - (uint32_t)m) : 0;
    if (out_val) out_val[t] = m ? __uint_as_float(((uint32_t)(m >> 32) & 0x80000000u) ? ((uint32_t)(m >> 32) & 0x7FFFFFFFu) : ~(uint32_t)(m >> 32))
                                : -INFINITY;
  }
}

}  // namespace qws

extern "C" size_t qws_head_ws_bytes(void) { return qws::HqLayout::total; }
extern "C" const int* qws_head_ws_cand(const void* ws) { return (const int*)((const char*)ws + qws::HqLayout::cand); }
extern "C" const float* qws_head_ws_exact(const void* ws) { return (const float*)((const char*)ws + qws::HqLayout::exact); }

extern "C" int qws_head_select_rescore(float* logits, const void* w_bf16, const void* x, int N, int K, int T, int R, int* out_tok, float* out_val, void* ws,
                                       void* stream, const int* ids) {
  using namespace qws;
  if (!logits || !w_bf16 || !x || !out_tok || !ws || ((uintptr_t)ws & 255) || ((uintptr_t)logits & 15) || ((uintptr_t)w_bf16 & 15) ||
      ((uintptr_t)x & 15))
    return QWS_ERR_INVALID;
  if (T < 1 || T > HQ_ROWS || R < 1 || R > HQ_RMAX || N < 4 || (N & 3) || K < 8 || (K & 7)) return QWS_ERR_INVALID;
  const int nch = (N + HQ_CHUNK - 1) / HQ_CHUNK;
  if (nch > HQ_NCH) return QWS_ERR_NOT_SUPPORTED;
  char* b = (char*)ws;
  int* cnt = (int*)(b + HqLayout::cnt);
  uint32_t* cm = (uint32_t*)(b + HqLayout::cm);
  int* cand = (int*)(b + HqLayout::cand);
  float* exact = (float*)(b + HqLayout::exact);
  uint64_t* list = (uint64_t*)(b + HqLayout::list);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_hq_chunkmax, dim3(nch, T), dim3(256), 0, st, logits, N, cm, cnt);
  hipLaunchKernelGGL(k_hq_extract, dim3(nch, T), dim3(256), 0, st, logits, N, R, cm, cnt, list);
  hipLaunchKernelGGL(k_hq_rank, dim3(T), dim3(512), 0, st, R, cnt, list, cand);
  hipLaunchKernelGGL(k_hq_rescore, dim3((R + 3) / 4, T), dim3(256), 0, st, (const uint4*)w_bf16, (const uint4*)x, N, K, R, logits, cand, exact, ids);
  hipLaunchKernelGGL(k_hq_argmax, dim3(T), dim3(64), 0, st, R, cand, exact, ids, out_tok, out_val);
  return (int)hipGetLastError();
}
