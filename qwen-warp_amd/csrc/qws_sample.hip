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

// The small fields of a chunk record, staged in LDS by the resolver (one coalesced copy instead of dependent
// global loads inside serial loops).
struct HS {
  uint32_t max_key, max_idx;
  int nexp, n_cand, n_win, n_gath, n_iv, top_set;
  int ivlo[MAXIV], ivhi[MAXIV];
  uint32_t cnt_part[MAXIV];
  uint64_t mu_part[MAXIV];
};
__device__ inline void stage_heads(char* ws, const Layout& L, int row, HS* hs) {
  for (int g = threadIdx.x; g < L.G; g += NT) {
    const Head* H = head_of(ws, L, row, g);
    HS h;
    h.max_key = H->max_key;
    h.max_idx = H->max_idx;
    h.nexp = H->nexp;
    h.n_cand = H->n_cand;
    h.n_win = H->n_win;
    h.n_gath = H->n_gath;
    h.n_iv = H->n_iv;
    h.top_set = H->top_set;
    for (int k = 0; k < MAXIV; k++) {
      h.ivlo[k] = H->iv[k].lo;
      h.ivhi[k] = H->iv[k].hi;
      h.cnt_part[k] = H->iv[k].cnt_part;
      h.mu_part[k] = H->iv[k].mu_part;
    }
    hs[g] = h;
  }
  __syncthreads();
}

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

__device__ inline float kappa_of(const qws_row& R) { return kappa_f(R.temperature); }

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
// hist word of a fine bin: (count << 40) | summed mantissas (< 2^38 for a chunk of <= 2^14 elements)
constexpr int HC_SHIFT = 40;
constexpr unsigned long long HM_MASK = (1ull << HC_SHIFT) - 1;

template <typename T>
__device__ inline T wave_scan_incl(T v) {  // inclusive prefix over lanes
  const int lane = lane_id();
  for (int o = 1; o < 64; o <<= 1) {
    const T u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}
__device__ inline int first_lane(bool p) {  // lowest lane with p, or 64
  const unsigned long long b = __ballot(p);
  return b ? __ffsll((long long)b) - 1 : 64;
}

// The first pass's view of its chunk histogram, evaluated by one wave.  Top-down positions: t = NBIN - 1 - bin;
// exponent u = t >> 6 from the top (u = 0 holds the chunk's best candidate).  cc / cm: inclusive per-exponent
// prefix (counts, approximate masses) held by lane u.
struct WaveView {
  const unsigned long long* hist;
  uint32_t cc;   // lane u: elements in exponents 0..u
  float cm;      // lane u: approximate mass in exponents 0..u (relative to the chunk's top power of two)
  __device__ inline uint32_t ccof(int u) const { return u < 0 ? 0u : (uint32_t)__shfl((int)cc, u < NEXP ? u : NEXP - 1, 64); }
  __device__ inline float cmof(int u) const { return u < 0 ? 0.0f : __shfl(cm, u < NEXP ? u : NEXP - 1, 64); }
  // fine bin of top-down position (u, lane): bin = NBIN - 1 - (u * 64 + lane)
  __device__ inline unsigned long long h(int u, int lane) const { return hist[NBIN - 1 - (u * FB + lane)]; }
  // elements at top-down positions [0, t]
  __device__ inline uint32_t cnt_to(int t) const {
    if (t < 0) return 0u;
    if (t >= NBIN) t = NBIN - 1;
    const int u = t >> 6, lane = lane_id();
    const uint32_t c = lane <= (t & 63) ? (uint32_t)(h(u, lane) >> HC_SHIFT) : 0u;
    return ccof(u - 1) + wave_sum<uint32_t>(c);
  }
  __device__ inline float mass_to(int t) const {
    if (t < 0) return 0.0f;
    if (t >= NBIN) t = NBIN - 1;
    const int u = t >> 6, lane = lane_id();
    const float m = lane <= (t & 63) ? ldexpf((float)(h(u, lane) & HM_MASK), -u - 23) : 0.0f;
    return cmof(u - 1) + wave_sum<float>(m);
  }
  // first top-down position whose inclusive count reaches target (NBIN if none)
  __device__ inline int count_cross(uint32_t target) const {
    const int u = first_lane(lane_id() < NEXP && cc >= target);
    if (u >= NEXP) return NBIN;
    const uint32_t c = wave_scan_incl<uint32_t>((uint32_t)(h(u, lane_id()) >> HC_SHIFT)) + ccof(u - 1);
    const int l = first_lane(c >= target);
    return u * FB + (l < 64 ? l : 63);
  }
  __device__ inline int mass_cross(float target) const {
    const int u = first_lane(lane_id() < NEXP && cm >= target);
    if (u >= NEXP) return NBIN;
    const float m = wave_scan_incl<float>(ldexpf((float)(h(u, lane_id()) & HM_MASK), -u - 23)) + cmof(u - 1);
    const int l = first_lane(m >= target);
    return u * FB + (l < 64 ? l : 63);
  }
};

template <int E, int DT>
__global__ void __launch_bounds__(NT) k_first(qws_batch B, Layout L, char* ws) {
  constexpr int C = NT * E;
  static_assert(C - 256 >= 0, "exp2 table in the table array");
  __shared__ __attribute__((aligned(16))) uint32_t tab[C];   // processor table, then the exp2 table
  __shared__ unsigned long long hist[NBIN];
  __shared__ unsigned long long s_best;
  __shared__ int s_cnt, s_n;
  __shared__ int s_iv[2 * MAXIV];

  const int row = blockIdx.x / L.G, g = blockIdx.x % L.G;
  const int lo = g * C, hi = min(B.V, lo + C);
  const qws_row R = B.rows[row];
  Head* H = head_of(ws, L, row, g);
  uint64_t* EL = elems_of(ws, L, row, g);
  float* etab = (float*)(tab + C - 256);
  if (threadIdx.x == 0) {
    s_cnt = 0;
    s_best = 0ull;
  }
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
  // best candidate (a thread's elements come in increasing index: keep the first of equal keys) and candidates
  uint32_t bk = 0, bi = 0, nc = 0;
#pragma unroll
  for (int e = 0; e < E; e++) {
    const uint32_t k = okey(x[e]);
    const bool better = k > bk;
    bi = better ? (uint32_t)elt_index<E, DT>(lo, e) : bi;
    bk = better ? k : bk;
    nc += x[e] != -INFINITY;
  }
  const uint64_t wb = wave_max_u64(bk ? comp(bk, bi) : 0ull);
  nc = wave_sum<uint32_t>(nc);
  __syncthreads();  // every thread is done with the processor table
  if (lane_id() == 0) {
    atomicMax((unsigned long long*)&s_best, (unsigned long long)wb);
    atomicAdd(&s_cnt, (int)nc);
  }
  for (int b = threadIdx.x; b < NBIN; b += NT) hist[b] = 0ull;
  if (threadIdx.x < 256) etab[threadIdx.x] = __uint_as_float(EXP2_TAB[threadIdx.x]);
  __syncthreads();
  const uint64_t best = s_best;
  const int tot = s_cnt;
  const uint32_t max_key = (uint32_t)(best >> 32), max_idx = 0xFFFFFFFFu - (uint32_t)best;
  if (!(R.temperature > 0.0f) || tot == 0) {
    if (threadIdx.x == 0) {
      H->max_key = max_key;
      H->max_idx = max_idx;
      H->n_cand = tot;
      H->n_win = 0;
      H->n_gath = 0;
      H->n_iv = 0;
      H->top_set = 0;
      H->nexp = 0;
    }
    return;
  }
  const float kappa = kappa_of(R);
  const float amax = log2u(okey_val(max_key), kappa);
  const int Ng = weigh(amax, etab).n();
  const int base = (Ng - D_EXP) * FB;
  int rb[E];
#pragma unroll
  for (int e = 0; e < E; e++) {
    const W w = weigh(log2u(x[e], kappa), etab);
    const int r = w.bin() - base;
    rb[e] = (x[e] != -INFINITY && r >= 0) ? r : -1;  // r < NBIN: the chunk's best candidate is in exponent Ng
    if (rb[e] >= 0) atomicAdd(&hist[r], (1ull << HC_SHIFT) | (unsigned long long)w.mu);
  }
  __syncthreads();
  // per-exponent record, wave per power of two (e = 38 is the top)
  for (int e = wave_id(); e < NEXP; e += NWAVE) {
    const unsigned long long h = hist[e * FB + lane_id()];
    const unsigned long long c = wave_sum<unsigned long long>(h >> HC_SHIFT);
    const unsigned long long m = wave_sum<unsigned long long>(h & HM_MASK);
    if (lane_id() == 0) {
      H->ccnt[e] = (uint32_t)c;
      H->cmu[e] = m;
    }
  }
  // ---- wave 0: the resolver's needs and the intervals handed over
  if (wave_id() == 0) {
    const int lane = lane_id();
    WaveView vw;
    vw.hist = hist;
    {  // per-exponent inclusive prefix from the top, lane u = exponent 38 - u
      const unsigned long long h0 = 0;
      uint32_t c = 0;
      float m = 0.0f;
      if (lane < NEXP) {
        const int e = D_EXP - lane;
        for (int b = 0; b < FB; b++) {  // 64 bins of this lane's exponent (conflict-free: lanes read distinct banks in turn)
          const unsigned long long h = hist[e * FB + ((b + lane) & 63)];
          c += (uint32_t)(h >> HC_SHIFT);
          m += (float)(h & HM_MASK);
        }
        m = ldexpf(m, -lane - 23);
      }
      (void)h0;
      vw.cc = wave_scan_incl<uint32_t>(c);
      vw.cm = wave_scan_incl<float>(m);
    }
    const uint32_t ctot = vw.ccof(NEXP - 1);
    constexpr uint32_t TOPB = 128;
    constexpr int MARGIN = 6;
    const bool topk = R.top_k > 0, topp = R.top_p < 1.0f, minp = R.min_p > 0.0f;
    int t_m = NBIN - 1;
    if (minp) {  // the row's best is at least the chunk's: its min_p cut lies at or above this one
      const int rc = weigh((float)((double)amax + R.log2_min_p), etab).bin() - base;
      t_m = rc < 0 ? NBIN - 1 : NBIN - 1 - rc;
    }
    int t_k = NBIN - 1;
    if (topk) {
      const uint32_t tgt = (uint32_t)(R.top_k <= 64 ? R.top_k : min(R.top_k, 2 * R.top_k / L.G + 64));
      t_k = min(vw.count_cross(tgt), NBIN - 1);
    }
    const int t_b = vw.count_cross(TOPB + 1) - 1;  // deepest position with at most TOPB elements at or above it
    const int t_lim = min(t_k, t_m);
    int t_p = NBIN - 1;
    if (topp) t_p = min(vw.mass_cross(R.top_p * vw.mass_to(t_lim)), t_lim);
    int floor_t = -1;  // top set = top-down positions [0, floor_t]
    if (topk && vw.cnt_to(t_k) <= CAP) floor_t = max(floor_t, t_k);
    if (minp && vw.cnt_to(t_m) <= CAP) floor_t = max(floor_t, t_m);
    const int t_nuc = min(NBIN - 1, t_p + MARGIN);
    if (topp && vw.cnt_to(t_nuc) <= CAP) floor_t = max(floor_t, t_nuc);
    if (topp) floor_t = max(floor_t, min(t_b, NBIN - 1));
    int niv = 0;
    uint32_t used = 0;
    if (floor_t >= 0) {
      if (lane == 0) {
        H->iv[0].lo = NBIN - 1 - floor_t;
        H->iv[0].hi = NBIN - 1;
        H->iv[0].cnt_part = 0;
        H->iv[0].mu_part = 0;
        H->iv[0].pad = 0;
        s_iv[0] = NBIN - 1 - floor_t;
        s_iv[1] = NBIN - 1;
      }
      used = vw.cnt_to(floor_t);
      niv = 1;
    }
    if (topp && t_nuc > floor_t) {  // a window around the local top-p boundary
      for (int m = MARGIN; m >= 0; m--) {
        const int a = max(floor_t + 1, t_p - m), b = min(NBIN - 1, t_p + m);
        if (a > b) break;
        const uint32_t n = vw.cnt_to(b) - vw.cnt_to(a - 1);
        if (used + n <= CAP) {
          const int vlo = NBIN - 1 - b, vhi = NBIN - 1 - a;
          // elements above vhi inside vhi's power of two: top-down positions [u * 64, a - 1] of exponent u = a >> 6
          const int u = a >> 6;
          const unsigned long long hh = (lane < (a & 63)) ? vw.h(u, lane) : 0ull;
          const unsigned long long cp = wave_sum<unsigned long long>(hh >> HC_SHIFT);
          const unsigned long long mp = wave_sum<unsigned long long>(hh & HM_MASK);
          if (lane == 0) {
            H->iv[niv].lo = vlo;
            H->iv[niv].hi = vhi;
            H->iv[niv].cnt_part = (uint32_t)cp;
            H->iv[niv].mu_part = mp;
            H->iv[niv].pad = 0;
            s_iv[2 * niv] = vlo;
            s_iv[2 * niv + 1] = vhi;
          }
          niv++;
          used += n;
          break;
        }
      }
    }
    if (lane == 0) {
      H->max_key = max_key;
      H->max_idx = max_idx;
      H->nexp = Ng;
      H->n_cand = tot;
      H->n_win = (int)ctot;
      H->n_iv = niv;
      H->top_set = floor_t >= 0;
      s_n = niv;
      s_cnt = 0;  // gather counter
    }
  }
  __syncthreads();
  const int niv = s_n;
  int ivlo[MAXIV], ivhi[MAXIV];
#pragma unroll
  for (int k = 0; k < MAXIV; k++) {
    ivlo[k] = k < niv ? s_iv[2 * k] : 1;
    ivhi[k] = k < niv ? s_iv[2 * k + 1] : 0;
  }
#pragma unroll
  for (int e = 0; e < E; e++) {
    const int r = rb[e];
    bool take = false;
#pragma unroll
    for (int k = 0; k < MAXIV; k++) take |= r >= ivlo[k] && r <= ivhi[k];
    if (r >= 0 && take) {
      const int pos = atomicAdd(&s_cnt, 1);
      if (pos < CAP) EL[pos] = ((uint64_t)okey(x[e]) << 32) | (uint64_t)(uint32_t)elt_index<E, DT>(lo, e);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) H->n_gath = min(s_cnt, CAP);
}

// ---------------------------------------------------------------------------------------------- resolver
// LDS pool of k_resolve (bytes): [tab: C * 4][region X: 3 * XN * 8][bcnt, boff: 2 * NBK * 4]
constexpr int XN = 2048;                                   // elements per LDS element buffer
constexpr size_t POOL_X = 3ull * XN * 8;                   // three element buffers (or a level-1 histogram)
static_assert(NBIN * 12 <= (int)POOL_X, "level-1 histogram fits region X");

struct RowState {          // per-row state of k_resolve (LDS)
  int G, C, V;
  uint32_t max_key, max_idx;
  float kappa, a_max, a_cut;  // a_cut: min_p keeps candidates with a >= a_cut
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
  const float a = log2u(okey_val(key), st.kappa);
  *mp = !st.minp || a >= st.a_cut;
  return wunits(weigh_c(a), st.N);
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
// Without a cut or min_p, a chunk's kept mass is its whole window mass, exact from its first-pass record
// (wave per chunk, lane per power of two).
template <int E, int DT>
__device__ int draw_row(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, const RowState& st, const HS* hs, uint64_t cut,
                        u128 S2, uint32_t u24, const Pool& P, u128* Mg) {
  const u128 t = ((u128)u24 * S2) >> 24;
  if (cut == 0 && !st.minp) {
    const int w = wave_id(), lane = lane_id();
    for (int g = w; g < st.G; g += NWAVE) {
      const Head* H = head_of(ws, L, row, g);
      u128 m = 0;
      if (hs[g].n_win && lane < NEXP) {
        const int sh = hs[g].nexp - D_EXP + lane - (st.N - D_EXP);
        if (sh >= 0) m = (u128)H->cmu[lane] << sh;
      }
      m = wave_sum_u128(m);
      if (lane == 0) Mg[g] = m;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      u128 c = 0;
      P.si[4] = -1;
      for (int g = 0; g < st.G; g++) {
        if (t < c + Mg[g]) {
          P.si[4] = g;
          P.su[0] = t - c;
          break;
        }
        c += Mg[g];
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
      const float a = log2u(x, st.kappa);
      if (st.minp && !(a >= st.a_cut)) return;
      const W w = weigh_c(a);
      const long long rb = (long long)w.bin() - wbase;
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
        const float a = log2u(x, st.kappa);
        if (st.minp && !(a >= st.a_cut)) return;
        const W w = weigh_c(a);
        if ((long long)w.bin() != bin_abs) return;
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
        const float a = log2u(x, st.kappa);
        if (st.minp && !(a >= st.a_cut)) return;
        const W w = weigh_c(a);
        if ((long long)w.bin() != bin_abs) return;
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
__device__ int merge_row(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, RowState& st, HS* hs, const Pool& P) {
  constexpr int C = NT * E;
  const int G = L.G;
  stage_heads(ws, L, row, hs);
  uint64_t best = 0;
  int ncand = 0;
  for (int g = threadIdx.x; g < G; g += NT) {
    const uint64_t c = comp(hs[g].max_key, hs[g].max_idx);
    best = c > best ? c : best;
    ncand += hs[g].n_cand;
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
    st.N = weigh_c(st.a_max).n();
    st.topp = R.top_p < 1.0f;
    st.a_cut = (float)((double)st.a_max + R.log2_min_p);
    // min_p cuts into the weight window only when a_cut lies above its floor
    st.minp = R.min_p > 0.0f && st.a_cut > (float)(st.N - D_EXP);
  }
  if (threadIdx.x < NEXP) {
    st.gcnt[threadIdx.x] = 0u;
    st.gmu[threadIdx.x] = 0ull;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < G * NEXP; p += NT) {
    const int g = p / NEXP, e = p % NEXP;
    if (hs[g].n_win == 0) continue;
    const int ge = hs[g].nexp - D_EXP + e - (st.N - D_EXP);
    if (ge >= 0 && ge < NEXP) {
      const Head* H = head_of(ws, L, row, g);
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

// ---------------------------------------------------------------------------------------------- runs resolver
// Every chunk handed over its elements in a few bin intervals (absolute fine bins), plus exact per-exponent sums
// and, per interval, the sum of the elements above it inside its top power of two.  The bins every chunk covers
// form "runs"; inside a run all elements are known, and the exact mass / count above the run is known.  The
// top-k, min-p and top-p boundaries are located bin by bin inside the runs and element by element inside one bin.
constexpr int MAXR = 4;
struct Runs {
  int n;
  long long lo[MAXR], hi[MAXR];  // absolute bins, descending runs
  u128 cam[MAXR];                // exact mass above each run (units 2^(N - 38 - 23))
  unsigned long long cac[MAXR];  // count above each run
  long long base;                // absolute bin of the window floor, (N - 38) * 64
};
struct Loc {
  long long bin;
  u128 cm;                       // mass before the bin (rank order)
  unsigned long long cc;         // count before the bin
  int ok;
};
struct Cut {
  uint64_t c;                    // comp of the last kept element
  u128 cm;                       // inclusive mass at it
  unsigned long long cc;         // inclusive count at it
  int ok;
};

__device__ inline void iv_abs(const HS& H, int k, long long* lo, long long* hi) {
  const long long b = ((long long)H.nexp - D_EXP) * FB;
  *lo = b + H.ivlo[k];
  *hi = (k == 0 && H.top_set) ? LLONG_MAX : b + H.ivhi[k];
}
// interval of chunk H that contains [lo, hi], or -1
__device__ inline int iv_containing(const HS& H, long long lo, long long hi) {
  for (int k = 0; k < H.n_iv; k++) {
    long long a, b;
    iv_abs(H, k, &a, &b);
    if (a <= lo && hi <= b) return k;
  }
  return -1;
}
__device__ inline long long fdiv64(long long b) { return b >= 0 ? b / FB : -((-b + FB - 1) / FB); }

// Exact (mass, count) of chunk H's elements above interval k's top, computed by the 64 lanes of a wave
// (lane e < 39 handles exponent nexp - 38 + e).  Top-set intervals have nothing above them.
__device__ inline void above_iv(const HS& H, const Head* Hg, int k, int N, u128* m, unsigned long long* c) {
  u128 lm = 0;
  unsigned long long lc = 0;
  if (!(k == 0 && H.top_set)) {
    long long lo, hi;
    iv_abs(H, k, &lo, &hi);
    const long long Ehi = fdiv64(hi);
    const int e = lane_id();
    if (e < NEXP) {
      const long long n = (long long)H.nexp - D_EXP + e;
      if (n > Ehi && n >= N - D_EXP) {
        lm = (u128)Hg->cmu[e] << (int)(n - (N - D_EXP));
        lc = Hg->ccnt[e];
      }
    }
    if (e == 0 && Ehi >= N - D_EXP) {
      lm += (u128)H.mu_part[k] << (int)(Ehi - (N - D_EXP));
      lc += H.cnt_part[k];
    }
  }
  *m = wave_sum_u128(lm);
  *c = wave_sum<unsigned long long>(lc);
}

__device__ inline long long elem_bin(uint64_t v, const RowState& st, uint64_t* w) {
  const float a = log2u(okey_val((uint32_t)(v >> 32)), st.kappa);
  const W ww = weigh_c(a);
  *w = wunits(ww, st.N);
  return (long long)ww.bin();
}

// Runs = bins every chunk with window candidates covers, clamped to the weight window.  Thread 0.
__device__ void build_runs(const Layout& L, const HS* hs, const RowState& st, Runs& R) {
  long long lo[MAXR * 4], hi[MAXR * 4];
  int n = 1;
  lo[0] = ((long long)st.N - D_EXP) * FB;
  hi[0] = (long long)weigh_c(st.a_max).bin();
  for (int g = 0; g < L.G && n > 0; g++) {
    const HS& H = hs[g];
    if (H.n_win == 0) continue;
    long long nlo[MAXR * 4], nhi[MAXR * 4];
    int m = 0;
    for (int i = 0; i < n; i++)
      for (int k = 0; k < H.n_iv; k++) {
        long long a, b;
        iv_abs(H, k, &a, &b);
        const long long x = a > lo[i] ? a : lo[i], y = b < hi[i] ? b : hi[i];
        if (x <= y && m < MAXR * 4) {
          nlo[m] = x;
          nhi[m] = y;
          m++;
        }
      }
    n = m;
    for (int i = 0; i < m; i++) {
      lo[i] = nlo[i];
      hi[i] = nhi[i];
    }
  }
  // keep the highest MAXR runs, descending
  for (int i = 0; i < n; i++)
    for (int j = i + 1; j < n; j++)
      if (hi[j] > hi[i]) {
        long long t = hi[i]; hi[i] = hi[j]; hi[j] = t;
        t = lo[i]; lo[i] = lo[j]; lo[j] = t;
      }
  R.n = n < MAXR ? n : MAXR;
  for (int i = 0; i < R.n; i++) {
    R.lo[i] = lo[i];
    R.hi[i] = hi[i];
  }
  R.base = ((long long)st.N - D_EXP) * FB;
}

// Flat, parallel iteration over every element the first pass handed over for this row.  goff: prefix offsets
// of the chunks' element counts (LDS, G + 1 entries); an element's chunk is its token index / C.
template <typename F>
__device__ inline void for_gathered(const Layout& L, char* ws, int row, const int* goff, F fn) {
  const int n = goff[L.G];
  int g = 0;
  constexpr int U = 4;
  for (int i0 = threadIdx.x; i0 < n; i0 += U * NT) {
    uint64_t v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * NT;
      v[u] = 0;
      if (i < n) {
        while (goff[g + 1] <= i) g++;
        v[u] = elems_of(ws, L, row, g)[i - goff[g]];
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (i0 + u * NT < n) fn(v[u]);
  }
}

// Exact (mass, count) of chunk g's elements above interval k's top (one thread; the 39 record loads are independent).
__device__ inline void above_serial(const HS& H, const Head* Hg, int k, int N, u128* m, unsigned long long* c) {
  u128 lm = 0;
  unsigned long long lc = 0;
  if (!(k == 0 && H.top_set)) {
    long long lo, hi;
    iv_abs(H, k, &lo, &hi);
    const long long Ehi = fdiv64(hi);
    for (int e = 0; e < NEXP; e++) {
      const long long n = (long long)H.nexp - D_EXP + e;
      if (n > Ehi && n >= N - D_EXP) {
        lm += (u128)Hg->cmu[e] << (int)(n - (N - D_EXP));
        lc += Hg->ccnt[e];
      }
    }
    if (Ehi >= N - D_EXP) {
      lm += (u128)H.mu_part[k] << (int)(Ehi - (N - D_EXP));
      lc += H.cnt_part[k];
    }
  }
  *m = lm;
  *c = lc;
}

struct RunTabs {               // per (chunk, run), LDS
  long long hi[MAXG * MAXR];   // top of the chunk's interval that contains the run
  u128 am[MAXG * MAXR];        // exact mass above that interval
  unsigned long long ac[MAXG * MAXR];
};

// Exact mass / count above each run, and per-bin sums inside the runs, from every handed-over element.
__device__ void runs_pass(const Layout& L, char* ws, int row, const HS* hs, const int* goff, const RowState& st, Runs& R, RunTabs& T,
                          unsigned long long* binm, uint32_t* binc, u128* red128) {
  for (int b = threadIdx.x; b < NBIN; b += NT) {
    binm[b] = 0ull;
    binc[b] = 0u;
  }
  for (int p = threadIdx.x; p < L.G * MAXR; p += NT) {
    const int g = p / MAXR, r = p % MAXR;
    T.hi[p] = LLONG_MIN;
    T.am[p] = 0;
    T.ac[p] = 0;
    if (r >= R.n || hs[g].n_win == 0) continue;
    const int k = iv_containing(hs[g], R.lo[r], R.hi[r]);
    if (k < 0) continue;
    long long a;
    iv_abs(hs[g], k, &a, &T.hi[p]);
    above_serial(hs[g], head_of(ws, L, row, g), k, st.N, &T.am[p], &T.ac[p]);
  }
  __syncthreads();
  const int C = st.C;
  u128 am[MAXR] = {0, 0, 0, 0};
  unsigned long long ac[MAXR] = {0, 0, 0, 0};
  for_gathered(L, ws, row, goff, [&](uint64_t v) {
    const int g = (int)((uint32_t)v / (uint32_t)C);
    uint64_t wt;
    const float a = log2u(okey_val((uint32_t)(v >> 32)), st.kappa);
    const W ww = weigh_c(a);
    const long long b = ww.bin();
    wt = wunits(ww, st.N);
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
      if (r >= R.n) break;
      if (b > R.hi[r] && b <= T.hi[g * MAXR + r]) {
        am[r] += wt;
        ac[r] += 1;
      }
      if (b >= R.lo[r] && b <= R.hi[r]) {
        const int rb = (int)(b - R.base);
        atomicAdd(&binm[rb], (unsigned long long)ww.mu);
        atomicAdd(&binc[rb], 1u);
      }
    }
  });
  for (int r = 0; r < MAXR; r++) {
    u128 m = am[r], c = ac[r];
    for (int g = threadIdx.x; g < L.G; g += NT) {
      m += T.am[g * MAXR + r];
      c += T.ac[g * MAXR + r];
    }
    m = block_sum_u128(m, red128);
    c = block_sum_u128(c, red128);
    if (threadIdx.x == 0 && r < R.n) {
      R.cam[r] = m;
      R.cac[r] = (unsigned long long)c;
    }
  }
  __syncthreads();
}

// The bin inside the runs where the cumulative (rank order) count / mass first reaches target, or a given bin
// (want_bin >= 0): its cumulative mass and count before it.
__device__ Loc locate(const Runs& R, const unsigned long long* binm, const uint32_t* binc, int by_mass, u128 target, long long want_bin,
                      u128* red128, u128* s_top, Loc* s_loc) {
  constexpr int PP = (NBIN + NT - 1) / NT;
  u128 vm[PP], vc[PP];
  u128 lm = 0, lc = 0;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k;
    vm[k] = 0;
    vc[k] = 0;
    if (t < NBIN) {
      const int b = NBIN - 1 - t;
      vm[k] = (u128)binm[b] << (b >> 6);
      vc[k] = binc[b];
    }
    lm += vm[k];
    lc += vc[k];
  }
  u128 tm, tc;
  const u128 im = block_scan_u128(lm, red128, &tm);
  const u128 ic = block_scan_u128(lc, red128, &tc);
  if (threadIdx.x == 0) s_loc->ok = 0;
  // prefix before each run's top bin
  u128 pm = im - lm, pc = ic - lc;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k;
    const long long b = R.base + (NBIN - 1 - t);
    for (int r = 0; r < R.n; r++)
      if (b == R.hi[r]) {
        s_top[2 * r] = pm;
        s_top[2 * r + 1] = pc;
      }
    pm += vm[k];
    pc += vc[k];
  }
  __syncthreads();
  pm = im - lm;
  pc = ic - lc;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k;
    const long long b = R.base + (NBIN - 1 - t);
    for (int r = 0; r < R.n; r++) {
      if (b < R.lo[r] || b > R.hi[r]) continue;
      const u128 bm = R.cam[r] + pm - s_top[2 * r];
      const u128 bc = (u128)R.cac[r] + pc - s_top[2 * r + 1];
      const u128 before = by_mass ? bm : bc;
      const u128 after = before + (by_mass ? vm[k] : vc[k]);
      const bool hit = want_bin >= 0 ? (b == want_bin + 0) : (before < target && after >= target);
      if (hit) {
        s_loc->bin = b;
        s_loc->cm = bm;
        s_loc->cc = (unsigned long long)bc;
        s_loc->ok = 1;
      }
    }
    pm += vm[k];
    pc += vc[k];
  }
  __syncthreads();
  const Loc out = *s_loc;
  __syncthreads();
  return out;
}

// Inside bin b (covered by every chunk): the first element in rank order whose inclusive cumulative count /
// mass reaches target, starting from (cm, cc) before the bin.  Elements failing min_p weigh and count 0.
// target = 0 with by_mass = 2 walks the whole bin (returns its min_p-passing totals).
__device__ Cut walk_bin(const Layout& L, char* ws, int row, const HS* hs, const int* goff, const qws_row& Rw, const RowState& st, long long bin,
                        u128 cm, unsigned long long cc, int by_mass, u128 target, const Pool& P) {
  Cut out = {0, 0, 0, 0};
  (void)hs;
  if (threadIdx.x == 0) P.si[1] = 0;
  __syncthreads();
  for_gathered(L, ws, row, goff, [&](uint64_t v) {
    uint64_t wt;
    if (elem_bin(v, st, &wt) != bin) return;
    const int pos = atomicAdd(&P.si[1], 1);
    if (pos < XN) P.ea[pos] = comp((uint32_t)(v >> 32), (uint32_t)v);
  });
  __syncthreads();
  const int n = P.si[1];
  __syncthreads();
  if (n > XN) return out;
  if (n > 0) lds_sort_desc(P.ea, P.eb, n, P);
  const int Q = (n + NT - 1) / NT;
  const int j0 = threadIdx.x * Q, j1 = min(n, j0 + Q);
  u128 lm = 0, lc = 0;
  for (int j = j0; j < j1; j++) {
    const uint64_t wt = dom_weight((uint32_t)(P.ea[j] >> 32), st, Rw);
    lm += wt;
    lc += wt ? 1 : 0;
  }
  u128 tm, tc;
  const u128 im = block_scan_u128(lm, P.red128, &tm);
  const u128 ic = block_scan_u128(lc, P.red128, &tc);
  if (by_mass == 2) {
    out.c = 0;
    out.cm = cm + tm;
    out.cc = cc + (unsigned long long)tc;
    out.ok = 1;
    return out;
  }
  if (threadIdx.x == 0) P.si[2] = -1;
  __syncthreads();
  u128 m = cm + im - lm, c = (u128)cc + ic - lc;
  for (int j = j0; j < j1; j++) {
    const uint64_t wt = dom_weight((uint32_t)(P.ea[j] >> 32), st, Rw);
    const u128 m2 = m + wt, c2 = c + (wt ? 1 : 0);
    const u128 before = by_mass ? m : c, after = by_mass ? m2 : c2;
    if (wt && before < target && after >= target) {
      P.si[2] = j;
      P.su[0] = m2;
      P.su[1] = c2;
    }
    m = m2;
    c = c2;
  }
  __syncthreads();
  const int js = P.si[2];
  if (js >= 0) {
    out.c = P.ea[js];
    out.cm = P.su[0];
    out.cc = (unsigned long long)P.su[1];
    out.ok = 1;
  }
  __syncthreads();
  return out;
}

// Kept mass of every chunk (elements with comp >= cut in the domain), given the bin of the cut.
__device__ void chunk_masses(const Layout& L, char* ws, int row, const HS* hs, const int* goff, const qws_row& Rw, const RowState& st,
                             long long bin_c, uint64_t cut, u128* Mg, unsigned long long* mlo, unsigned long long* mhi, long long* chi) {
  for (int g = threadIdx.x; g < L.G; g += NT) {
    u128 m = 0;
    chi[g] = LLONG_MIN;
    if (hs[g].n_win) {
      const int k = iv_containing(hs[g], bin_c, bin_c);
      if (k >= 0) {
        long long a;
        iv_abs(hs[g], k, &a, &chi[g]);
        unsigned long long c;
        above_serial(hs[g], head_of(ws, L, row, g), k, st.N, &m, &c);
      }
    }
    mlo[g] = (unsigned long long)m;
    mhi[g] = (unsigned long long)(m >> 64);
  }
  __syncthreads();
  const int C = st.C;
  for_gathered(L, ws, row, goff, [&](uint64_t v) {
    const int g = (int)((uint32_t)v / (uint32_t)C);
    uint64_t wt;
    const long long b = elem_bin(v, st, &wt);
    uint64_t add = 0;
    if (b > bin_c && b <= chi[g]) add = wt;
    else if (b == bin_c && comp((uint32_t)(v >> 32), (uint32_t)v) >= cut) add = dom_weight((uint32_t)(v >> 32), st, Rw);
    if (add) {
      const unsigned long long old = atomicAdd(&mlo[g], (unsigned long long)add);
      if (old + add < old) atomicAdd(&mhi[g], 1ull);
    }
  });
  __syncthreads();
  for (int g = threadIdx.x; g < L.G; g += NT) Mg[g] = ((u128)mhi[g] << 64) | mlo[g];
  __syncthreads();
}

// Resolves a sampling row from the first-pass records.  Returns 1 when the token is written, 0 when a boundary
// lies outside the handed-over bins (the caller then rescans).
template <int E, int DT>
__device__ int resolve_runs(const qws_batch& B, const qws_row& Rw, int row, const Layout& L, char* ws, const RowState& st, const HS* hs,
                            const int* goff, uint32_t u24, const Pool& P, Runs& R, RunTabs& T, Loc* s_loc, u128* s_top, u128* Mg,
                            unsigned long long* mlo, unsigned long long* mhi, long long* chi) {
  unsigned long long* binm = (unsigned long long*)P.tab;
  uint32_t* binc = (uint32_t*)((char*)P.tab + NBIN * 8);
  if (threadIdx.x == 0) build_runs(L, hs, st, R);
  __syncthreads();
  if (R.n == 0) return 0;
  runs_pass(L, ws, row, hs, goff, st, R, T, binm, binc, P.red128);
  // ---- min_p: the domain ends inside the cut bin
  bool minp = st.minp;
  long long bm_bin = 0;
  u128 Dm = st.S_all;
  unsigned long long Dc = st.n_win;
  if (minp) {
    bm_bin = (long long)weigh_c(st.a_cut).bin();
    if (bm_bin < R.base) {
      minp = false;  // every window element passes
    } else {
      const Loc lb = locate(R, binm, binc, 1, 0, bm_bin, P.red128, s_top, s_loc);
      if (!lb.ok) return 0;
      const Cut t = walk_bin(L, ws, row, hs, goff, Rw, st, bm_bin, lb.cm, lb.cc, 2, 0, P);
      if (!t.ok) return 0;
      Dm = t.cm;
      Dc = t.cc;
    }
  }
  // ---- top-k
  long long bin_c = -1;
  uint64_t cut = 0;
  u128 S = Dm;
  bool have_cut = false;
  if (Rw.top_k > 0 && (unsigned long long)Rw.top_k < Dc) {
    const Loc lk = locate(R, binm, binc, 0, (u128)Rw.top_k, -1, P.red128, s_top, s_loc);
    if (!lk.ok) return 0;
    const Cut ck = walk_bin(L, ws, row, hs, goff, Rw, st, lk.bin, lk.cm, lk.cc, 0, (u128)Rw.top_k, P);
    if (!ck.ok) return 0;
    bin_c = lk.bin;
    cut = ck.c;
    S = ck.cm;
    have_cut = true;
  }
  // ---- top-p
  if (st.topp) {
    const u128 TP = (u128)(uint64_t)floor((double)Rw.top_p * 4294967296.0);
    const u128 thr = (TP * S + (((u128)1 << 32) - 1)) >> 32;
    const Loc lp = locate(R, binm, binc, 1, thr, -1, P.red128, s_top, s_loc);
    if (!lp.ok) return 0;
    const Cut cp = walk_bin(L, ws, row, hs, goff, Rw, st, lp.bin, lp.cm, lp.cc, 1, thr, P);
    if (!cp.ok) return 0;
    bin_c = lp.bin;
    cut = cp.c;
    S = cp.cm;
    have_cut = true;
  }
  if (!have_cut) {
    if (!minp) return 0;  // nothing selects: the pure path handles it
    bin_c = bm_bin;
    cut = 0;
  }
  // ---- draw: chunk by kept mass, then inside the chunk
  chunk_masses(L, ws, row, hs, goff, Rw, st, bin_c, cut, Mg, mlo, mhi, chi);
  const u128 t = ((u128)u24 * S) >> 24;
  if (threadIdx.x == 0) {
    u128 c = 0;
    P.si[4] = -1;
    for (int g = 0; g < L.G; g++) {
      if (t < c + Mg[g]) {
        P.si[4] = g;
        P.su[2] = t - c;
        break;
      }
      c += Mg[g];
    }
  }
  __syncthreads();
  const int gs = P.si[4];
  const u128 tl = P.su[2];
  __syncthreads();
  if (gs < 0) return 0;
  const int tok = draw_in_chunk<E, DT>(B, Rw, row, gs, st, cut, tl, P);
  if (tok < 0) return 0;
  if (B.out_probs) write_probs<E, DT>(B, Rw, row, st, cut, S, P);
  if (threadIdx.x == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = 0;
  }
  return 1;
}

template <int E, int DT>
__global__ void __launch_bounds__(NT) k_resolve(qws_batch B, Layout L, char* ws) {
  constexpr int C = NT * E;
  constexpr int TABB = (C * 4 > NBIN * 12 ? C * 4 : NBIN * 12);
  __shared__ __attribute__((aligned(16))) unsigned char pool[TABB + POOL_X + 2 * NBK * 4];
  __shared__ Runs runs;
  __shared__ Loc s_loc;
  __shared__ u128 s_top[2 * MAXR];
  __shared__ u128 Mg[MAXG];
  __shared__ HS hs[MAXG];
  __shared__ RunTabs rtab;
  __shared__ int goff[MAXG + 1];
  __shared__ unsigned long long mlo[MAXG], mhi[MAXG];
  __shared__ long long chi[MAXG];
  __shared__ uint64_t red64[NWAVE];
  __shared__ u128 red128[NWAVE];
  __shared__ uint32_t redu[NWAVE];
  __shared__ int si[8];
  __shared__ u128 su[4];
  __shared__ uint64_t sc[4];
  __shared__ RowState st;
  Pool P;
  P.tab = (uint32_t*)pool;
  P.ea = (uint64_t*)(pool + TABB);
  P.eb = P.ea + XN;
  P.ec = P.eb + XN;
  P.hc = (uint32_t*)(pool + TABB);
  P.hm = (unsigned long long*)(pool + TABB + ((NBIN * 4 + 15) & ~15));
  P.bcnt = (uint32_t*)(pool + TABB + POOL_X);
  P.boff = P.bcnt + NBK;
  P.red64 = red64;
  P.red128 = red128;
  P.redu = redu;
  P.si = si;
  P.su = su;
  P.sc = sc;

  const int row = blockIdx.x;
  const qws_row R = B.rows[row];
  if (!merge_row<E>(B, R, row, L, ws, st, hs, P)) return;
  const uint32_t u24 = draw_u24(R.seed, R.position, R.stream, R.row_key, 0);
  if (st.topk || st.minp || st.topp) {
    if (threadIdx.x == 0) {
      int o = 0;
      for (int g = 0; g < L.G; g++) {
        goff[g] = o;
        o += hs[g].n_gath;
      }
      goff[L.G] = o;
    }
    __syncthreads();
    if (resolve_runs<E, DT>(B, R, row, L, ws, st, hs, goff, u24, P, runs, rtab, &s_loc, s_top, Mg, mlo, mhi, chi)) return;
    __syncthreads();
  }
  // ---- exact resolution by rescans (also the path of pure temperature sampling)
  uint64_t cut = 0;
  u128 S = st.S_all;
  int info = 1;
  bool ok = true;
  if (!(st.topk || st.minp || st.topp)) info = 3;  // nothing to select: the first-pass records suffice
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
  if (ok) tok = draw_row<E, DT>(B, R, row, L, ws, st, hs, cut, S, u24, P, Mg);
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
  (void)B;
  (void)V;
  return 8;  // 4,096-token chunks: 36 KB of LDS, four workgroups per CU
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
