// qws sampling kernels for MI355X (gfx950).
//
// One call samples B rows of V logits in two launches:
//   k_first   (B x G workgroups, one per chunk of C tokens): one streaming pass over the logits.  It
//             applies the request processors, finds the chunk's best candidate, histograms the fixed-point
//             weights by absolute fine bin (exact per-power-of-two sums, mergeable across chunks
//             without knowing the row maximum) and hands the resolver the chunk's candidates that the
//             row's top-k / min-p / top-p decisions can depend on.
//   k_resolve (B workgroups, one per row): merges the G chunk records, resolves greedy / min-p / top-k /
//             top-p exactly and draws the token (Philox4x32-10, inverse CDF in index order).  Whatever
//             the first pass did not hand over is recomputed exactly by rescanning chunks.
// The definition being computed is stated in oracle/sampler.py; the reference it restates is
// engine/src/proc.h:39-49 (processors), engine/src/mtp_sample.cu:122-183 (temperature / min_p / top-k /
// top-p), engine/src/mtp_sample.cu:10-27 (Philox draw) and engine/src/misc.cu:50-111 (argmax).
#include <math.h>
#include <stdlib.h>

#include "qws_device.h"

namespace qws {

constexpr int ECAP = 3072;   // candidate elements the resolver holds in LDS
constexpr int NBK = 2048;    // buckets of the LDS sort / digit histograms

struct IV {                  // a bin interval [lo, hi] (bins relative to the chunk window) handed over completely
  int lo, hi;
  uint32_t cnt_part;         // elements above hi inside hi's power of two
  uint32_t pad;
  uint64_t mu_part;          // their summed mantissas
};
struct Head {                // one chunk's record, written by k_first
  uint32_t max_key, max_idx; // best candidate (key, lowest index)
  int nexp;                  // floor(a) of the chunk's best candidate: window = exponents [nexp - 38, nexp]
  int n_cand;                // finite candidates
  int n_win;                 // candidates inside the window
  int n_gath;                // elements handed over
  int n_iv;                  // intervals; iv[0] is the top set when top_set != 0
  int top_set;               // 1: iv[0] = [lo, NBIN - 1] (everything from lo up)
  IV iv[MAXIV];
  uint32_t ccnt[NEXP];       // per-exponent counts of the window
  uint32_t pad2;
  uint64_t cmu[NEXP];        // per-exponent summed mantissas
};
constexpr size_t HEAD_BYTES = (sizeof(Head) + 255) & ~(size_t)255;

struct Layout {
  int G, C;                  // chunks per row, tokens per chunk
  size_t rec_bytes;          // bytes per (row, chunk) record: head + CAP elements
};
__device__ inline Head* head_of(char* ws, const Layout& L, int row, int g) { return (Head*)(ws + ((size_t)row * L.G + g) * L.rec_bytes); }
__device__ inline uint64_t* elems_of(char* ws, const Layout& L, int row, int g) { return (uint64_t*)(ws + ((size_t)row * L.G + g) * L.rec_bytes + HEAD_BYTES); }

// ---------------------------------------------------------------------------------------------- chunk processing
template <int DT>
struct Vec { static constexpr int N = DT == QWS_DTYPE_F32 ? 4 : 8; };

// element e of this thread: index lo + (e / VEC * NT + tid) * VEC + e % VEC
template <int E, int DT>
__device__ inline int elt_index(int lo, int e) {
  constexpr int VEC = Vec<DT>::N;
  return lo + ((e / VEC) * NT + (int)threadIdx.x) * VEC + (e % VEC);
}

// Per-chunk processor state: tab[token - lo] = count | bias slot | stop | prompt (engine/src/proc.cu:72-103
// builds the same state densely per request; here it is rebuilt per chunk from the row's history).
__device__ void build_table(const qws_batch& B, const qws_row& R, int lo, int hi, uint32_t* tab, int C) {
  for (int i = threadIdx.x; i < C; i += NT) tab[i] = 0u;
  __syncthreads();
  const int* h = B.hist + R.hist_off;
  for (int j = threadIdx.x; j < R.n_prompt; j += NT) {
    const int id = h[j];
    if (id >= lo && id < hi) atomicOr(&tab[id - lo], TB_PROMPT);
  }
  for (int j = threadIdx.x; j < R.n_gen; j += NT) {
    const int id = h[R.n_prompt + j];
    if (id >= lo && id < hi) atomicAdd(&tab[id - lo], 1u);
  }
  for (int j = threadIdx.x; j < R.n_drafts; j += NT) {
    const int id = B.drafts[R.draft_off + j];
    if (id >= lo && id < hi) atomicAdd(&tab[id - lo], 1u);
  }
  if (R.min_tokens > R.ngen + R.n_drafts) {
    for (int j = threadIdx.x; j < R.n_stop; j += NT) {
      const int id = B.stop_ids[R.stop_off + j];
      if (id >= lo && id < hi) atomicOr(&tab[id - lo], TB_STOP);
    }
  }
  for (int j = threadIdx.x; j < R.n_bias; j += NT) {
    const int id = B.bias_ids[R.bias_off + j];
    if (id >= lo && id < hi) atomicOr(&tab[id - lo], (uint32_t)(j + 1) << TB_SLOT_SHIFT);
  }
  __syncthreads();
}

// engine/src/proc.h:39-49, one IEEE rounding per operation
__device__ inline float proc_one(float x, uint32_t t, bool masked, const qws_row& R, const float* bias_row) {
  if (masked) x = -INFINITY;
  if (t & TB_STOP) x = -INFINITY;
  const uint32_t slot = (t >> TB_SLOT_SHIFT) & TB_SLOT;
  const float b = slot ? bias_row[slot - 1] : 0.0f;
  x = x + b;
  const uint32_t cnt = t & TB_CNT;
  if (R.repetition != 1.0f && ((t & TB_PROMPT) || cnt)) x = x > 0.0f ? x / R.repetition : x * R.repetition;
  if (cnt) {
    x = x - R.frequency * (float)cnt;
    x = x - R.presence;
  }
  return x;
}

__device__ inline float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Loads one chunk [lo, hi) of row `row` into x[E] (processed; -inf outside the chunk).  tab must hold the
// chunk's table when R.proc_on.
template <int E, int DT>
__device__ inline void load_chunk(const qws_batch& B, const qws_row& R, int row, int lo, int hi, const uint32_t* tab, float (&x)[E]) {
  constexpr int VEC = Vec<DT>::N;
  constexpr int S = E / VEC;
  const size_t esz = DT == QWS_DTYPE_F32 ? 4 : 2;
  const char* base = (const char*)B.logits + (size_t)row * (size_t)B.row_stride * esz;
#pragma unroll
  for (int s = 0; s < S; s++) {
    const int i0 = lo + (s * NT + (int)threadIdx.x) * VEC;
    if (i0 < hi) {
      if constexpr (DT == QWS_DTYPE_F32) {
        const float4 v = *(const float4*)(base + (size_t)i0 * 4);
        x[s * 4 + 0] = v.x; x[s * 4 + 1] = v.y; x[s * 4 + 2] = v.z; x[s * 4 + 3] = v.w;
      } else {
        const uint4 v = *(const uint4*)(base + (size_t)i0 * 2);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          x[s * 8 + 2 * j] = bf16f((uint16_t)(w[j] & 0xFFFFu));
          x[s * 8 + 2 * j + 1] = bf16f((uint16_t)(w[j] >> 16));
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; j++) x[s * VEC + j] = -INFINITY;
    }
  }
#pragma unroll
  for (int e = 0; e < E; e++) x[e] = x[e] != x[e] ? -INFINITY : x[e];
  if (!R.proc_on) return;
  const float* bias_row = B.bias_vals + R.bias_off;
  const unsigned* mrow = R.mask_mode ? B.masks + (size_t)R.mask_row * (size_t)B.mask_words : nullptr;
#pragma unroll
  for (int s = 0; s < S; s++) {
    const int i0 = lo + (s * NT + (int)threadIdx.x) * VEC;
    if (i0 >= hi) continue;
    const uint32_t mw = mrow ? mrow[i0 >> 5] : 0u;
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      const int i = i0 + j;
      const uint32_t bit = (mw >> (i & 31)) & 1u;
      const bool masked = R.mask_mode == QWS_MASK_BANNED ? bit != 0u : (R.mask_mode == QWS_MASK_ALLOWED ? bit == 0u : false);
      x[s * VEC + j] = proc_one(x[s * VEC + j], tab[i - lo], masked, R, bias_row);
    }
  }
}

__device__ inline double kappa_of(const qws_row& R) { return (double)(1.0f / R.temperature) * LOG2E; }

// ---------------------------------------------------------------------------------------------- small block scans
template <typename T>
__device__ inline T block_scan_incl(T v, T* red, T* total) {
  const int lane = lane_id(), w = wave_id();
  T s = v;
  for (int o = 1; o < 64; o <<= 1) {
    const T u = __shfl_up(s, o, 64);
    if (lane >= o) s += u;
  }
  __syncthreads();
  if (lane == 63) red[w] = s;
  __syncthreads();
  T before = 0, t = 0;
  for (int i = 0; i < NWAVE; i++) {
    if (i < w) before += red[i];
    t += red[i];
  }
  *total = t;
  return before + s;
}

// ---------------------------------------------------------------------------------------------- k_first
template <int E, int DT>
__global__ void __launch_bounds__(NT) k_first(qws_batch B, Layout L, char* ws) {
  constexpr int C = NT * E;
  constexpr int P = (NBIN + NT - 1) / NT;  // bins per thread in the top-down scans
  __shared__ uint32_t tab[C];
  __shared__ uint32_t hcnt[NBIN];
  __shared__ unsigned long long hmu[NBIN];
  __shared__ uint64_t red64[NWAVE];
  __shared__ double redd[NWAVE];
  __shared__ uint32_t redu[NWAVE];
  __shared__ int s_tk, s_tp, s_n;
  __shared__ double s_mass;

  const int row = blockIdx.x / L.G, g = blockIdx.x % L.G;
  const int lo = g * C, hi = min(B.V, lo + C);
  const qws_row R = B.rows[row];
  Head* H = head_of(ws, L, row, g);
  uint64_t* EL = elems_of(ws, L, row, g);

  if (R.proc_on) build_table(B, R, lo, hi, tab, C);
  float x[E];
  load_chunk<E, DT>(B, R, row, lo, hi, tab, x);
  if (B.out_logits) {
#pragma unroll
    for (int e = 0; e < E; e++) {
      const int i = elt_index<E, DT>(lo, e);
      if (i < hi) B.out_logits[(size_t)row * B.V + i] = x[e];
    }
  }
  // best candidate and candidate count
  uint64_t best = 0;
  uint32_t ncand = 0;
#pragma unroll
  for (int e = 0; e < E; e++) {
    const int i = elt_index<E, DT>(lo, e);
    if (i < hi) {
      const uint64_t c = comp(okey(x[e]), (uint32_t)i);
      best = c > best ? c : best;
      ncand += x[e] != -INFINITY;
    }
  }
  best = block_max_u64(best, red64);
  uint32_t tot;
  block_scan_incl<uint32_t>(ncand, redu, &tot);
  const uint32_t max_key = (uint32_t)(best >> 32), max_idx = 0xFFFFFFFFu - (uint32_t)best;
  const bool sampling = R.temperature > 0.0f && tot > 0;
  if (!sampling) {
    if (threadIdx.x == 0) {
      H->max_key = max_key;
      H->max_idx = max_idx;
      H->n_cand = (int)tot;
      H->n_win = 0;
      H->n_gath = 0;
      H->n_iv = 0;
      H->top_set = 0;
      H->nexp = 0;
    }
    return;
  }
  const double kappa = kappa_of(R);
  const int Ng = (int)floor(log2u(okey_val(max_key), kappa));
  const long long base = ((long long)Ng - D_EXP) * FB;
  for (int b = threadIdx.x; b < NBIN; b += NT) {
    hcnt[b] = 0u;
    hmu[b] = 0ull;
  }
  __syncthreads();
  int rb[E];
#pragma unroll
  for (int e = 0; e < E; e++) {
    rb[e] = -1;
    if (x[e] != -INFINITY) {
      const W w = weigh(log2u(x[e], kappa));
      const long long r = w.bin - base;
      if (r >= 0) {
        rb[e] = (int)r;  // r < NBIN: the chunk's best candidate is in exponent Ng
        atomicAdd(&hcnt[r], 1u);
        atomicAdd(&hmu[r], (unsigned long long)w.mu);
      }
    }
  }
  __syncthreads();
  // per-exponent record
  if (threadIdx.x < NEXP) {
    uint32_t c = 0;
    uint64_t m = 0;
    for (int b = threadIdx.x * FB; b < (threadIdx.x + 1) * FB; b++) {
      c += hcnt[b];
      m += hmu[b];
    }
    H->ccnt[threadIdx.x] = c;
    H->cmu[threadIdx.x] = m;
  }
  // top-down inclusive scans of counts and (approximate) masses; thread j owns top-down bins [j*P, j*P+P)
  uint32_t cc[P];
  double cm[P];
  uint32_t lc = 0;
  double lm = 0.0;
#pragma unroll
  for (int k = 0; k < P; k++) {
    const int t = threadIdx.x * P + k;
    const int b = NBIN - 1 - t;
    if (t < NBIN) {
      lc += hcnt[b];
      lm += (double)hmu[b] * ldexp(1.0, (b >> 6) - D_EXP);
    }
    cc[k] = lc;
    cm[k] = lm;
  }
  uint32_t ctot;
  double mtot;
  const uint32_t cinc = block_scan_incl<uint32_t>(lc, redu, &ctot);
  const double minc = block_scan_incl<double>(lm, redd, &mtot);
  const uint32_t cbefore = cinc - lc;
  const double mbefore = minc - lm;
#pragma unroll
  for (int k = 0; k < P; k++) {
    cc[k] += cbefore;
    cm[k] += mbefore;
  }
  __syncthreads();
  // store the inclusive top-down count prefix in hcnt (indexed by top-down position)
#pragma unroll
  for (int k = 0; k < P; k++) {
    const int t = threadIdx.x * P + k;
    if (t < NBIN) hcnt[t] = cc[k];
  }
  // needs of the resolver, as top-down positions (larger = deeper)
  const bool topk = R.top_k > 0;
  const bool minp = R.min_p > 0.0f && R.log2_min_p > -(double)(D_EXP + 1);
  const bool topp = R.top_p < 1.0f;
  int tgt_k = 0;
  if (topk) tgt_k = R.top_k <= 64 ? R.top_k : min(R.top_k, 2 * R.top_k / L.G + 64);
  if (threadIdx.x == 0) {
    s_tk = NBIN - 1;
    s_tp = NBIN - 1;
  }
  __syncthreads();
  if (topk) {
#pragma unroll
    for (int k = 0; k < P; k++) {
      const int t = threadIdx.x * P + k;
      const uint32_t prev = k ? cc[k - 1] : cbefore;
      if (t < NBIN && prev < (uint32_t)tgt_k && cc[k] >= (uint32_t)tgt_k) s_tk = t;
    }
  }
  int t_m = NBIN - 1;
  if (minp) {
    const double acut = log2u(okey_val(max_key), kappa) + R.log2_min_p;
    const long long rc = (long long)floor(acut * 64.0) - base;
    t_m = rc < 0 ? NBIN - 1 : (int)(NBIN - 1 - rc);
  }
  __syncthreads();
  const int t_lim = min(topk ? s_tk : NBIN - 1, minp ? t_m : NBIN - 1);
  // local mass of the locally kept bins and the local top-p boundary
  if (threadIdx.x == t_lim / P) s_mass = cm[t_lim % P];
  __syncthreads();
  if (topp) {
    const double thr = (double)R.top_p * s_mass;
#pragma unroll
    for (int k = 0; k < P; k++) {
      const int t = threadIdx.x * P + k;
      const double prev = k ? cm[k - 1] : mbefore;
      if (t <= t_lim && prev < thr && cm[k] >= thr) s_tp = t;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    constexpr int MARGIN = 6;
    auto cnt_to = [&](int t) -> uint32_t { return t < 0 ? 0u : hcnt[t < NBIN ? t : NBIN - 1]; };  // elements in top-down positions [0, t]
    int floor_t = -1;  // top set = top-down positions [0, floor_t]
    if (topk && cnt_to(s_tk) <= CAP) floor_t = max(floor_t, s_tk);
    if (minp && cnt_to(t_m) <= CAP) floor_t = max(floor_t, t_m);
    const int t_nuc = min(NBIN - 1, s_tp + MARGIN);
    if (topp && cnt_to(t_nuc) <= CAP) floor_t = max(floor_t, t_nuc);
    int niv = 0;
    uint32_t used = 0;
    IV iv[MAXIV];
    auto above = [&](IV& v) {  // elements above v.hi inside v.hi's power of two
      const int e = v.hi >> 6;
      const int top = e * FB + FB - 1;
      uint64_t m = 0;
      for (int b = v.hi + 1; b <= top; b++) m += hmu[b];
      const int th = NBIN - 1 - v.hi;      // top-down position of hi
      const int ttop = NBIN - 1 - top;     // top-down position of the exponent's top bin
      v.cnt_part = cnt_to(th - 1) - cnt_to(ttop - 1);
      v.mu_part = m;
      v.pad = 0;
    };
    if (floor_t >= 0) {
      iv[0].lo = NBIN - 1 - floor_t;
      iv[0].hi = NBIN - 1;
      iv[0].cnt_part = 0;
      iv[0].mu_part = 0;
      iv[0].pad = 0;
      used = cnt_to(floor_t);
      niv = 1;
    }
    if (topp && t_nuc > floor_t) {  // a window around the local top-p boundary
      for (int m = MARGIN; m >= 0; m--) {
        const int a = max(floor_t + 1, s_tp - m), b = min(NBIN - 1, s_tp + m);
        if (a > b) break;
        const uint32_t n = cnt_to(b) - cnt_to(a - 1);
        if (used + n <= CAP) {
          iv[niv].lo = NBIN - 1 - b;
          iv[niv].hi = NBIN - 1 - a;
          above(iv[niv]);
          niv++;
          used += n;
          break;
        }
      }
    }
    H->max_key = max_key;
    H->max_idx = max_idx;
    H->nexp = Ng;
    H->n_cand = (int)tot;
    H->n_win = (int)ctot;
    H->n_iv = niv;
    H->top_set = floor_t >= 0;
    for (int k = 0; k < niv; k++) H->iv[k] = iv[k];
    s_n = niv;
    for (int k = 0; k < niv; k++) {
      tab[2 * k] = (uint32_t)iv[k].lo;
      tab[2 * k + 1] = (uint32_t)iv[k].hi;
    }
    s_tk = 0;  // gather counter
  }
  __syncthreads();
  const int niv = s_n;
  int ivlo[MAXIV], ivhi[MAXIV];
  for (int k = 0; k < MAXIV; k++) {
    ivlo[k] = k < niv ? (int)tab[2 * k] : 1;
    ivhi[k] = k < niv ? (int)tab[2 * k + 1] : 0;
  }
#pragma unroll
  for (int e = 0; e < E; e++) {
    const int r = rb[e];
    bool take = false;
    for (int k = 0; k < MAXIV; k++) take |= r >= ivlo[k] && r <= ivhi[k];
    if (r >= 0 && take) {
      const int pos = atomicAdd(&s_tk, 1);
      if (pos < CAP) EL[pos] = ((uint64_t)okey(x[e]) << 32) | (uint64_t)(uint32_t)elt_index<E, DT>(lo, e);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) H->n_gath = min(s_tk, CAP);
}

// ---------------------------------------------------------------------------------------------- resolver
// LDS pool of k_resolve (bytes): [tab: C * 4][region X: 3 * XN * 8][bcnt, boff: 2 * NBK * 4]
constexpr int XN = 2048;                                   // elements per LDS element buffer
constexpr size_t POOL_X = 3ull * XN * 8;                   // three element buffers (or a level-1 histogram)
static_assert(NBIN * 12 <= (int)POOL_X, "level-1 histogram fits region X");

struct RowState {          // per-row state of k_resolve (LDS)
  int G, C, V;
  uint32_t max_key, max_idx;
  double kappa, a_max;
  int N;
  uint32_t gcnt[NEXP];
  unsigned long long gmu[NEXP];
  u128 S_all;
  uint32_t n_win;
  int topk, minp, topp;
};

struct Pool {              // views into the LDS pool
  uint32_t* tab;
  uint64_t *ea, *eb, *ec;  // region X as three element buffers
  uint32_t* hc;            // region X as a level-1 histogram: counts [NBIN]
  unsigned long long* hm;  //                                  mantissa sums [NBIN]
  uint32_t *bcnt, *boff;
  uint64_t* red64;
  u128* red128;
  uint32_t* redu;
  int* si;
  u128* su;
  uint64_t* sc;
};

// Sorts n distinct u64 values descending (n <= XN): bucket by value range, rank inside each bucket.
__device__ void lds_sort_desc(uint64_t* a, uint64_t* tmp, int n, const Pool& P) {
  uint64_t mn = ~0ull, mx = 0;
  for (int i = threadIdx.x; i < n; i += NT) {
    mn = a[i] < mn ? a[i] : mn;
    mx = a[i] > mx ? a[i] : mx;
  }
  mx = block_max_u64(mx, P.red64);
  mn = ~block_max_u64(~mn, P.red64);
  const uint64_t range = mx - mn;
  int sh = 0;
  while (sh < 64 && (range >> sh) >= (uint64_t)NBK) sh++;
  for (int i = threadIdx.x; i < NBK; i += NT) P.bcnt[i] = 0u;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += NT) atomicAdd(&P.bcnt[NBK - 1 - (int)((a[i] - mn) >> sh)], 1u);
  __syncthreads();
  constexpr int PB = NBK / NT;
  uint32_t loc[PB];
  uint32_t s = 0;
#pragma unroll
  for (int k = 0; k < PB; k++) {
    loc[k] = s;
    s += P.bcnt[threadIdx.x * PB + k];
  }
  uint32_t tot;
  const uint32_t inc = block_scan_incl<uint32_t>(s, P.redu, &tot);
#pragma unroll
  for (int k = 0; k < PB; k++) P.boff[threadIdx.x * PB + k] = loc[k] + inc - s;
  __syncthreads();
  for (int i = threadIdx.x; i < NBK; i += NT) P.bcnt[i] = 0u;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += NT) {
    const int b = NBK - 1 - (int)((a[i] - mn) >> sh);
    tmp[P.boff[b] + atomicAdd(&P.bcnt[b], 1u)] = a[i];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += NT) {
    const uint64_t v = tmp[i];
    const int b = NBK - 1 - (int)((v - mn) >> sh);
    const int o = (int)P.boff[b], c = (int)P.bcnt[b];
    int r = o;
    for (int j = o; j < o + c; j++) r += tmp[j] > v;
    a[r] = v;
  }
  __syncthreads();
}

__device__ inline double u128_to_double(u128 v) { return (double)(uint64_t)(v >> 64) * 18446744073709551616.0 + (double)(uint64_t)v; }

// weight (units of 2^(N - 38 - 23)) of a key; *mp = passes min_p
__device__ inline uint64_t key_weight(uint32_t key, const RowState& st, const qws_row& R, bool* mp) {
  const double a = log2u(okey_val(key), st.kappa);
  *mp = !st.minp || (a - st.a_max) >= R.log2_min_p;
  return wunits(weigh(a), st.N);
}
// domain weight: > 0 only for candidates above the weight window floor that pass min_p
__device__ inline uint64_t dom_weight(uint32_t key, const RowState& st, const qws_row& R) {
  bool mp;
  const uint64_t w = key_weight(key, st, R, &mp);
  return mp ? w : 0ull;
}

// Calls fn(e, index, x) for every finite candidate of chunk g (rebuilding the chunk's processor table).
template <int E, int DT, typename F>
__device__ inline void for_chunk(const qws_batch& B, const qws_row& R, int row, int g, const RowState& st, const Pool& P, F fn) {
  const int lo = g * st.C, hi = min(st.V, lo + st.C);
  if (R.proc_on) build_table(B, R, lo, hi, P.tab, st.C);
  float x[E];
  load_chunk<E, DT>(B, R, row, lo, hi, P.tab, x);
#pragma unroll
  for (int e = 0; e < E; e++) {
    const int i = elt_index<E, DT>(lo, e);
    if (i < hi && x[e] != -INFINITY) fn(e, i, x[e]);
  }
  __syncthreads();
}

// Inverse CDF in index order inside chunk g over the kept set (domain weight > 0 and comp >= cut):
// the element whose kept-prefix interval contains t_local.  Returns the token or -1.
template <int E, int DT>
__device__ int draw_in_chunk(const qws_batch& B, const qws_row& R, int row, int g, const RowState& st, uint64_t cut, u128 t_local, const Pool& P) {
  constexpr int VEC = Vec<DT>::N;
  constexpr int S = E / VEC;
  const int lo = g * st.C, hi = min(st.V, lo + st.C);
  if (R.proc_on) build_table(B, R, lo, hi, P.tab, st.C);
  float x[E];
  load_chunk<E, DT>(B, R, row, lo, hi, P.tab, x);
  if (threadIdx.x == 0) P.si[7] = -1;
  __syncthreads();
  u128 run = 0;
  for (int s = 0; s < S; s++) {
    uint64_t w[VEC];
    uint64_t loc = 0;
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      const int e = s * VEC + j;
      const int i = elt_index<E, DT>(lo, e);
      w[j] = 0;
      if (i < hi && x[e] != -INFINITY) {
        const uint32_t k = okey(x[e]);
        if (comp(k, (uint32_t)i) >= cut) w[j] = dom_weight(k, st, R);
      }
      loc += w[j];
    }
    u128 tot;
    const u128 inc = block_scan_u128((u128)loc, P.red128, &tot);
    u128 c = run + inc - loc;
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      const u128 c2 = c + w[j];
      if (w[j] && c <= t_local && t_local < c2) P.si[7] = elt_index<E, DT>(lo, s * VEC + j);
      c = c2;
    }
    run += tot;
  }
  __syncthreads();
  const int tok = P.si[7];
  __syncthreads();
  return tok;
}

// Kept mass of chunk g (domain weight, comp >= cut).
template <int E, int DT>
__device__ u128 chunk_mass(const qws_batch& B, const qws_row& R, int row, int g, const RowState& st, uint64_t cut, const Pool& P) {
  u128 loc = 0;
  for_chunk<E, DT>(B, R, row, g, st, P, [&](int, int i, float x) {
    const uint32_t k = okey(x);
    if (comp(k, (uint32_t)i) >= cut) loc += dom_weight(k, st, R);
  });
  return block_sum_u128(loc, P.red128);
}

// Dense probabilities of the kept set (test-hook path).
template <int E, int DT>
__device__ void write_probs(const qws_batch& B, const qws_row& R, int row, const RowState& st, uint64_t cut, u128 S2, const Pool& P) {
  const double S2d = u128_to_double(S2);
  for (int g = 0; g < st.G; g++) {
    for_chunk<E, DT>(B, R, row, g, st, P, [&](int, int i, float x) {
      const uint32_t k = okey(x);
      if (comp(k, (uint32_t)i) < cut) return;
      const uint64_t w = dom_weight(k, st, R);
      if (w) B.out_probs[(size_t)row * st.V + i] = (float)((double)w / S2d);
    });
  }
}

// Draw over the whole row's kept set (mass S2): find the chunk by its kept mass, then the token inside it.
// Without a cut or min_p, a chunk's kept mass is its whole window mass, exact from its first-pass record.
template <int E, int DT>
__device__ int draw_row(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, const RowState& st, uint64_t cut, u128 S2,
                        uint32_t u24, const Pool& P) {
  const u128 t = ((u128)u24 * S2) >> 24;
  if (cut == 0 && !st.minp) {
    if (threadIdx.x == 0) {
      u128 c = 0;
      P.si[4] = -1;
      for (int g = 0; g < st.G; g++) {
        const Head* H = head_of(ws, L, row, g);
        u128 m = 0;
        if (H->n_win) {
          for (int e = 0; e < NEXP; e++) {
            const int sh = H->nexp - D_EXP + e - (st.N - D_EXP);
            if (sh >= 0) m += (u128)H->cmu[e] << sh;
          }
        }
        if (t < c + m) {
          P.si[4] = g;
          P.su[0] = t - c;
          break;
        }
        c += m;
      }
    }
    __syncthreads();
    const int g = P.si[4];
    const u128 tl = P.su[0];
    __syncthreads();
    return g < 0 ? -1 : draw_in_chunk<E, DT>(B, R, row, g, st, cut, tl, P);
  }
  u128 c = 0;
  for (int g = 0; g < st.G; g++) {
    const u128 m = chunk_mass<E, DT>(B, R, row, g, st, cut, P);
    if (t < c + m) return draw_in_chunk<E, DT>(B, R, row, g, st, cut, t - c, P);
    c += m;
  }
  return -1;
}

struct Sel {
  uint64_t c;       // comp of the selected element
  u128 cnt, mass;   // inclusive cumulative count / mass at it
  int ok;
};

// Exact selection by rescans: the first domain element in comp order (descending) whose inclusive
// cumulative count (by_mass = 0) or mass (by_mass = 1) reaches target.
template <int E, int DT>
__device__ Sel select_rescan(const qws_batch& B, const qws_row& R, int row, const RowState& st, int by_mass, u128 target, const Pool& P) {
  Sel out = {0, 0, 0, 0};
  const long long wbase = ((long long)st.N - D_EXP) * FB;
  // ---- level 1: histogram over the weight window's bins
  for (int b = threadIdx.x; b < NBIN; b += NT) {
    P.hc[b] = 0u;
    P.hm[b] = 0ull;
  }
  __syncthreads();
  for (int g = 0; g < st.G; g++) {
    for_chunk<E, DT>(B, R, row, g, st, P, [&](int, int, float x) {
      const double a = log2u(x, st.kappa);
      if (st.minp && !((a - st.a_max) >= R.log2_min_p)) return;
      const W w = weigh(a);
      const long long rb = w.bin - wbase;
      if (rb < 0) return;
      atomicAdd(&P.hc[rb], 1u);
      atomicAdd(&P.hm[rb], (unsigned long long)w.mu);
    });
  }
  // top-down scan: thread j owns top-down positions [j * PP, j * PP + PP)
  constexpr int PP = (NBIN + NT - 1) / NT;
  u128 mc[PP], cc[PP];
  u128 lm = 0, lc = 0;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k;
    if (t < NBIN) {
      const int b = NBIN - 1 - t;
      lc += P.hc[b];
      lm += (u128)P.hm[b] << (b >> 6);
    }
    cc[k] = lc;
    mc[k] = lm;
  }
  u128 tm, tc;
  const u128 im = block_scan_u128(lm, P.red128, &tm);
  const u128 ic = block_scan_u128(lc, P.red128, &tc);
  if (threadIdx.x == 0) P.si[0] = -1;
  __syncthreads();
  u128 pm = im - lm, pc = ic - lc;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k;
    const u128 vm = pm + mc[k], vc = pc + cc[k];
    const u128 before = by_mass ? pm + (k ? mc[k - 1] : 0) : pc + (k ? cc[k - 1] : 0);
    const u128 after = by_mass ? vm : vc;
    if (t < NBIN && before < target && after >= target) {
      P.si[0] = NBIN - 1 - t;
      P.su[0] = pm + (k ? mc[k - 1] : 0);  // mass above the bin
      P.su[1] = pc + (k ? cc[k - 1] : 0);  // count above the bin
    }
  }
  __syncthreads();
  const int bsel = P.si[0];
  if (bsel < 0) return out;
  u128 mass_above = P.su[0], cnt_above = P.su[1];
  __syncthreads();
  const long long bin_abs = wbase + bsel;
  // ---- inside the bin: narrow a comp range [cmin, cmax] until the set fits an LDS buffer
  uint64_t cmin = 0, cmax = ~0ull;
  for (int level = 0; level < 12; level++) {
    if (threadIdx.x == 0) {
      P.si[1] = 0;
      P.sc[0] = ~0ull;
      P.sc[1] = 0ull;
    }
    __syncthreads();
    // gather (up to XN elements) and the exact range of the set
    for (int g = 0; g < st.G; g++) {
      for_chunk<E, DT>(B, R, row, g, st, P, [&](int, int i, float x) {
        const double a = log2u(x, st.kappa);
        if (st.minp && !((a - st.a_max) >= R.log2_min_p)) return;
        const W w = weigh(a);
        if (w.bin != bin_abs) return;
        const uint64_t c = comp(okey(x), (uint32_t)i);
        if (c < cmin || c > cmax) return;
        const int pos = atomicAdd(&P.si[1], 1);
        if (pos < XN) P.ea[pos] = c;
        atomicMin((unsigned long long*)&P.sc[0], (unsigned long long)c);
        atomicMax((unsigned long long*)&P.sc[1], (unsigned long long)c);
      });
    }
    const int n = P.si[1];
    cmin = P.sc[0];
    cmax = P.sc[1];
    __syncthreads();
    if (n <= XN) {
      // walk the set in comp order
      lds_sort_desc(P.ea, P.eb, n, P);
      const int Q = (n + NT - 1) / NT;
      const int j0 = threadIdx.x * Q, j1 = min(n, j0 + Q);
      u128 loc = 0;
      for (int j = j0; j < j1; j++) loc += by_mass ? (u128)dom_weight((uint32_t)(P.ea[j] >> 32), st, R) : (u128)1;
      u128 tot;
      const u128 inc = block_scan_u128(loc, P.red128, &tot);
      u128 cum = (by_mass ? mass_above : cnt_above) + inc - loc;
      if (threadIdx.x == 0) P.si[2] = -1;
      __syncthreads();
      for (int j = j0; j < j1; j++) {
        const u128 c2 = cum + (by_mass ? (u128)dom_weight((uint32_t)(P.ea[j] >> 32), st, R) : (u128)1);
        if (cum < target && c2 >= target) P.si[2] = j;
        cum = c2;
      }
      __syncthreads();
      const int js = P.si[2];
      if (js < 0) return out;
      // cumulative count and mass at js
      u128 lmass = 0, lcnt = 0;
      for (int j = j0; j < min(j1, js + 1); j++) {
        lmass += dom_weight((uint32_t)(P.ea[j] >> 32), st, R);
        lcnt += 1;
      }
      const u128 sm = block_sum_u128(lmass, P.red128);
      const u128 sn = block_sum_u128(lcnt, P.red128);
      out.c = P.ea[js];
      out.mass = mass_above + sm;
      out.cnt = cnt_above + sn;
      out.ok = 1;
      __syncthreads();
      return out;
    }
    // too many: one digit level over [cmin, cmax]
    const uint64_t range = cmax - cmin;
    int sh = 0;
    while (sh < 64 && (range >> sh) >= (uint64_t)NBK) sh++;
    uint32_t* dc = P.bcnt;
    unsigned long long* dm = (unsigned long long*)P.eb;  // NBK mantissa sums (eb unused here)
    for (int d = threadIdx.x; d < NBK; d += NT) {
      dc[d] = 0u;
      dm[d] = 0ull;
    }
    __syncthreads();
    for (int g = 0; g < st.G; g++) {
      for_chunk<E, DT>(B, R, row, g, st, P, [&](int, int i, float x) {
        const double a = log2u(x, st.kappa);
        if (st.minp && !((a - st.a_max) >= R.log2_min_p)) return;
        const W w = weigh(a);
        if (w.bin != bin_abs) return;
        const uint64_t c = comp(okey(x), (uint32_t)i);
        if (c < cmin || c > cmax) return;
        const int d = NBK - 1 - (int)((c - cmin) >> sh);  // 0 = largest
        atomicAdd(&dc[d], 1u);
        atomicAdd(&dm[d], (unsigned long long)w.mu);
      });
    }
    const int e_sh = (int)(bin_abs >> 6) - (st.N - D_EXP);  // the bin's power of two inside the window
    if (threadIdx.x == 0) {
      u128 cm = mass_above, cn = cnt_above;
      int dsel = -1;
      for (int d = 0; d < NBK; d++) {
        const u128 m2 = cm + ((u128)dm[d] << e_sh), n2 = cn + dc[d];
        if ((by_mass ? m2 : n2) >= target && dc[d]) {
          dsel = d;
          break;
        }
        cm = m2;
        cn = n2;
      }
      P.si[3] = dsel;
      P.su[2] = cm;
      P.su[3] = cn;
    }
    __syncthreads();
    const int dsel = P.si[3];
    if (dsel < 0) return out;
    mass_above = P.su[2];
    cnt_above = P.su[3];
    const uint64_t dlo = cmin + ((uint64_t)(NBK - 1 - dsel) << sh);
    uint64_t dhi = dlo + ((1ull << sh) - 1);
    if (dhi < dlo || dhi > cmax) dhi = cmax;  // overflow or past the range
    cmin = dlo;
    cmax = dhi;
    __syncthreads();
  }
  return out;
}

// Merged per-row state from the chunk records.  Returns 0 when the row is greedy (token written).
template <int E>
__device__ int merge_row(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, RowState& st, const Pool& P) {
  constexpr int C = NT * E;
  const int G = L.G;
  uint64_t best = 0;
  int ncand = 0;
  for (int g = threadIdx.x; g < G; g += NT) {
    const Head* H = head_of(ws, L, row, g);
    const uint64_t c = comp(H->max_key, H->max_idx);
    best = c > best ? c : best;
    ncand += H->n_cand;
  }
  best = block_max_u64(best, P.red64);
  int ctot;
  block_scan_incl<int>(ncand, (int*)P.redu, &ctot);
  const uint32_t max_key = (uint32_t)(best >> 32), max_idx = 0xFFFFFFFFu - (uint32_t)best;
  if (!(R.temperature > 0.0f) || ctot == 0) {
    if (threadIdx.x == 0) {
      B.out_tokens[row] = (int)max_idx;
      if (B.out_info) B.out_info[row] = 2;
    }
    return 0;
  }
  if (threadIdx.x == 0) {
    st.G = G;
    st.C = C;
    st.V = B.V;
    st.max_key = max_key;
    st.max_idx = max_idx;
    st.kappa = kappa_of(R);
    st.a_max = log2u(okey_val(max_key), st.kappa);
    st.N = (int)floor(st.a_max);
    st.topp = R.top_p < 1.0f;
    st.minp = R.min_p > 0.0f && R.log2_min_p > -(double)(D_EXP + 1);
  }
  if (threadIdx.x < NEXP) {
    st.gcnt[threadIdx.x] = 0u;
    st.gmu[threadIdx.x] = 0ull;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < G * NEXP; p += NT) {
    const int g = p / NEXP, e = p % NEXP;
    const Head* H = head_of(ws, L, row, g);
    if (H->n_win == 0) continue;
    const int ge = H->nexp - D_EXP + e - (st.N - D_EXP);
    if (ge >= 0 && ge < NEXP) {
      atomicAdd(&st.gcnt[ge], H->ccnt[e]);
      atomicAdd(&st.gmu[ge], (unsigned long long)H->cmu[e]);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    u128 S = 0;
    uint32_t n = 0;
    for (int e = 0; e < NEXP; e++) {
      S += (u128)st.gmu[e] << e;
      n += st.gcnt[e];
    }
    st.S_all = S;
    st.n_win = n;
    st.topk = R.top_k > 0 && (uint32_t)R.top_k < n;
  }
  __syncthreads();
  return 1;
}

// Fast path: every element the kept set can contain was handed over by k_first.  Returns 1 when done.
template <int E, int DT>
__device__ int resolve_in_hand(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, const RowState& st, uint32_t u24, const Pool& P) {
  const int G = L.G;
  if (!(st.topk || st.minp || st.topp)) return 0;
  if (threadIdx.x == 0) P.si[0] = 1;
  __syncthreads();
  long long bs = LLONG_MIN;
  for (int g = threadIdx.x; g < G; g += NT) {
    const Head* H = head_of(ws, L, row, g);
    if (H->n_win == 0) continue;
    if (!H->top_set) P.si[0] = 0;
    else {
      const long long b = ((long long)H->nexp - D_EXP) * FB + H->iv[0].lo;
      bs = b > bs ? b : bs;
    }
  }
  const uint64_t enc = block_max_u64((uint64_t)bs ^ 0x8000000000000000ull, P.red64);
  if (!P.si[0]) return 0;
  const long long Bstar = (long long)(enc ^ 0x8000000000000000ull);
  if (threadIdx.x == 0) P.si[1] = 0;
  __syncthreads();
  for (int g = 0; g < G; g++) {
    const Head* H = head_of(ws, L, row, g);
    const int ng = H->n_gath;
    const uint64_t* EL = elems_of(ws, L, row, g);
    for (int j = threadIdx.x; j < ng; j += NT) {
      const uint64_t v = EL[j];
      const uint32_t k = (uint32_t)(v >> 32), idx = (uint32_t)v;
      const double a = log2u(okey_val(k), st.kappa);
      if ((long long)floor(a * 64.0) < Bstar) continue;
      if (st.minp && !((a - st.a_max) >= R.log2_min_p)) continue;
      const int pos = atomicAdd(&P.si[1], 1);
      if (pos < XN) P.ea[pos] = comp(k, idx);
    }
  }
  __syncthreads();
  const int n = P.si[1];
  __syncthreads();
  if (n > XN || n == 0) return 0;
  const long long cutbin = st.minp ? (long long)floor((st.a_max + R.log2_min_p) * 64.0) : LLONG_MIN;
  const bool minp_in_hand = st.minp && cutbin >= Bstar;
  if (st.topk && !(n >= R.top_k || minp_in_hand)) return 0;
  if (!st.topk && st.minp && !minp_in_hand) return 0;
  lds_sort_desc(P.ea, P.eb, n, P);
  const int nk = st.topk ? min(n, R.top_k) : n;
  const int Q = (nk + NT - 1) / NT;
  const int j0 = threadIdx.x * Q, j1 = min(nk, j0 + Q);
  u128 loc = 0;
  for (int j = j0; j < j1; j++) loc += dom_weight((uint32_t)(P.ea[j] >> 32), st, R);
  u128 tot;
  const u128 inc = block_scan_u128(loc, P.red128, &tot);
  const u128 S = (st.topk || st.minp) ? tot : st.S_all;
  int nkeep = nk;
  if (st.topp) {
    const u128 TP = (u128)(uint64_t)floor((double)R.top_p * 4294967296.0);
    const u128 thr = (TP * S + (((u128)1 << 32) - 1)) >> 32;
    if (threadIdx.x == 0) P.si[2] = -1;
    __syncthreads();
    u128 c = inc - loc;
    for (int j = j0; j < j1; j++) {
      const u128 c2 = c + dom_weight((uint32_t)(P.ea[j] >> 32), st, R);
      if (c < thr && c2 >= thr) P.si[2] = j;
      c = c2;
    }
    __syncthreads();
    if (P.si[2] < 0) return 0;  // the nucleus reaches below the handed-over set
    nkeep = P.si[2] + 1;
  }
  u128 l2 = 0;
  for (int j = j0; j < min(j1, nkeep); j++) l2 += dom_weight((uint32_t)(P.ea[j] >> 32), st, R);
  const u128 S2 = block_sum_u128(l2, P.red128);
  const u128 t = ((u128)u24 * S2) >> 24;
  // index order: (0xFFFFFFFF - idx) << 32 | rank, sorted descending = index ascending
  for (int j = threadIdx.x; j < nkeep; j += NT) P.eb[j] = ((uint64_t)(uint32_t)P.ea[j] << 32) | (uint64_t)j;
  __syncthreads();
  lds_sort_desc(P.eb, P.ec, nkeep, P);
  const int Q2 = (nkeep + NT - 1) / NT;
  const int q0 = threadIdx.x * Q2, q1 = min(nkeep, q0 + Q2);
  u128 lw = 0;
  for (int q = q0; q < q1; q++) lw += dom_weight((uint32_t)(P.ea[(uint32_t)P.eb[q]] >> 32), st, R);
  u128 tt;
  const u128 inc2 = block_scan_u128(lw, P.red128, &tt);
  u128 c = inc2 - lw;
  if (threadIdx.x == 0) P.si[3] = -1;
  __syncthreads();
  for (int q = q0; q < q1; q++) {
    const uint64_t w = dom_weight((uint32_t)(P.ea[(uint32_t)P.eb[q]] >> 32), st, R);
    const u128 c2 = c + w;
    if (w && c <= t && t < c2) P.si[3] = (int)(0xFFFFFFFFu - (uint32_t)(P.eb[q] >> 32));
    c = c2;
  }
  __syncthreads();
  if (B.out_probs) {
    const double S2d = u128_to_double(S2);
    for (int j = threadIdx.x; j < nkeep; j += NT) {
      const uint64_t w = dom_weight((uint32_t)(P.ea[j] >> 32), st, R);
      if (w) B.out_probs[(size_t)row * B.V + (0xFFFFFFFFu - (uint32_t)P.ea[j])] = (float)((double)w / S2d);
    }
  }
  if (threadIdx.x == 0) {
    B.out_tokens[row] = P.si[3];
    if (B.out_info) B.out_info[row] = 0;
  }
  return 1;
}

template <int E, int DT>
__global__ void __launch_bounds__(NT) k_resolve(qws_batch B, Layout L, char* ws) {
  constexpr int C = NT * E;
  __shared__ __attribute__((aligned(16))) unsigned char pool[C * 4 + POOL_X + 2 * NBK * 4];
  __shared__ uint64_t red64[NWAVE];
  __shared__ u128 red128[NWAVE];
  __shared__ uint32_t redu[NWAVE];
  __shared__ int si[8];
  __shared__ u128 su[4];
  __shared__ uint64_t sc[4];
  __shared__ RowState st;
  Pool P;
  P.tab = (uint32_t*)pool;
  P.ea = (uint64_t*)(pool + C * 4);
  P.eb = P.ea + XN;
  P.ec = P.eb + XN;
  P.hc = (uint32_t*)(pool + C * 4);
  P.hm = (unsigned long long*)(pool + C * 4 + ((NBIN * 4 + 15) & ~15));
  P.bcnt = (uint32_t*)(pool + C * 4 + POOL_X);
  P.boff = P.bcnt + NBK;
  P.red64 = red64;
  P.red128 = red128;
  P.redu = redu;
  P.si = si;
  P.su = su;
  P.sc = sc;

  const int row = blockIdx.x;
  const qws_row R = B.rows[row];
  if (!merge_row<E>(B, R, row, L, ws, st, P)) return;
  const uint32_t u24 = draw_u24(R.seed, R.position, R.stream, R.row_key, 0);
  if (resolve_in_hand<E, DT>(B, R, row, L, ws, st, u24, P)) return;
  __syncthreads();
  // ---- exact resolution by rescans (also the path of pure temperature sampling)
  uint64_t cut = 0;
  u128 S = st.S_all;
  int info = 1;
  bool ok = true;
  if (!(st.topk || st.minp || st.topp)) info = 0;  // nothing to select: the first-pass records suffice
  if (st.minp) {
    // domain mass with min_p: select with an unreachable target returns nothing but we need S; use the
    // count target n_win + 1 is unreachable, so compute S by one pass
    u128 loc = 0;
    for (int g = 0; g < st.G; g++) {
      for_chunk<E, DT>(B, R, row, g, st, P, [&](int, int, float x) { loc += dom_weight(okey(x), st, R); });
    }
    S = block_sum_u128(loc, P.red128);
  }
  if (st.topk) {
    const Sel s = select_rescan<E, DT>(B, R, row, st, 0, (u128)R.top_k, P);
    if (s.ok) {
      cut = s.c;
      S = s.mass;
    }  // else: fewer than K domain elements: top-k keeps them all
  }
  if (st.topp) {
    const u128 TP = (u128)(uint64_t)floor((double)R.top_p * 4294967296.0);
    const u128 thr = (TP * S + (((u128)1 << 32) - 1)) >> 32;
    const Sel s = select_rescan<E, DT>(B, R, row, st, 1, thr, P);
    if (s.ok) {
      cut = s.c;
      S = s.mass;
    } else {
      ok = false;
    }
  }
  int tok = -1;
  if (ok) tok = draw_row<E, DT>(B, R, row, L, ws, st, cut, S, u24, P);
  if (B.out_probs && ok) write_probs<E, DT>(B, R, row, st, cut, S, P);
  if (threadIdx.x == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = ok ? info : -1;
  }
}

}  // namespace qws

// ---------------------------------------------------------------------------------------------- launcher
namespace qws {
static int pick_E(int B, int V) {
  // more, smaller chunks when few rows would leave CUs idle
  const long long wg16 = (long long)B * ((V + NT * 16 - 1) / (NT * 16));
  return wg16 >= 512 ? 16 : 8;
}
static Layout layout_for(int B, int V, int E) {
  Layout L;
  L.C = NT * E;
  L.G = (V + L.C - 1) / L.C;
  L.rec_bytes = HEAD_BYTES + (size_t)CAP * 8;
  return L;
}
// Optional launch timing (profiling only): events recorded around each kernel of qws_sample.
struct Timing {
  bool on = false;
  int n = 0;
  static constexpr int CAPN = 4096;
  hipEvent_t ev[CAPN][3];
  bool made = false;
};
static Timing g_timing;

template <int E, int DT>
static hipError_t launch(const qws_batch& b, const Layout& L, char* ws, hipStream_t st) {
  const bool tm = g_timing.on && g_timing.n < Timing::CAPN;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][0], st);
  hipLaunchKernelGGL((k_first<E, DT>), dim3(b.B * L.G), dim3(NT), 0, st, b, L, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][1], st);
  hipLaunchKernelGGL((k_resolve<E, DT>), dim3(b.B), dim3(NT), 0, st, b, L, ws);
  e = hipGetLastError();
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n++][2], st);
  return e;
}
}  // namespace qws

extern "C" int qws_timing(int enable) {
  using namespace qws;
  if (enable && !g_timing.made) {
    for (int i = 0; i < Timing::CAPN; i++)
      for (int j = 0; j < 3; j++) {
        const hipError_t e = hipEventCreate(&g_timing.ev[i][j]);
        if (e != hipSuccess) return (int)e;
      }
    g_timing.made = true;
  }
  g_timing.on = enable != 0;
  g_timing.n = 0;
  return 0;
}

extern "C" int qws_timing_read(float* ms_first, float* ms_resolve, int* launches) {
  using namespace qws;
  float a = 0.f, r = 0.f;
  for (int i = 0; i < g_timing.n; i++) {
    hipError_t e = hipEventSynchronize(g_timing.ev[i][2]);
    if (e != hipSuccess) return (int)e;
    float x = 0.f, y = 0.f;
    e = hipEventElapsedTime(&x, g_timing.ev[i][0], g_timing.ev[i][1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&y, g_timing.ev[i][1], g_timing.ev[i][2]);
    if (e != hipSuccess) return (int)e;
    a += x;
    r += y;
  }
  *ms_first = a;
  *ms_resolve = r;
  *launches = g_timing.n;
  g_timing.n = 0;
  return 0;
}

extern "C" size_t qws_sample_ws_bytes(int B, int V) {
  if (B < 1 || V < 8) return 0;
  const qws::Layout L = qws::layout_for(B, V, 8);  // the larger of the two layouts
  return (size_t)B * L.G * L.rec_bytes;
}

extern "C" int qws_sample(const qws_batch* b, void* ws, size_t ws_bytes, void* stream) {
  using namespace qws;
  if (!b || !b->logits || !b->rows || !b->out_tokens || !ws) return QWS_ERR_INVALID;
  if (b->B < 1 || b->V < 8 || (b->V & 7) || (b->row_stride & 7) || b->row_stride < 0) return QWS_ERR_INVALID;
  if (b->row_stride != 0 && b->row_stride < b->V) return QWS_ERR_INVALID;
  if (b->dtype != QWS_DTYPE_F32 && b->dtype != QWS_DTYPE_BF16) return QWS_ERR_INVALID;
  if (((uintptr_t)b->logits & 15) || ((uintptr_t)ws & 255)) return QWS_ERR_INVALID;
  if (b->masks && b->mask_words * 32LL < b->V) return QWS_ERR_INVALID;
  const int E = pick_E(b->B, b->V);
  const Layout L = layout_for(b->B, b->V, E);
  if (L.G > MAXG) return QWS_ERR_NOT_SUPPORTED;
  if (ws_bytes < (size_t)b->B * L.G * L.rec_bytes) return QWS_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  char* w = (char*)ws;
  hipError_t e;
  if (b->dtype == QWS_DTYPE_F32) e = E == 16 ? launch<16, QWS_DTYPE_F32>(*b, L, w, st) : launch<8, QWS_DTYPE_F32>(*b, L, w, st);
  else e = E == 16 ? launch<16, QWS_DTYPE_BF16>(*b, L, w, st) : launch<8, QWS_DTYPE_BF16>(*b, L, w, st);
  return (int)e;
}
