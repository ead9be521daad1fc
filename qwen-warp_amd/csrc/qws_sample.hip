// qws sampling kernels for MI355X (gfx950).
//
// One call samples B rows of V logits in two launches:
//   k_first   (B x G workgroups, one per chunk of 4,096 tokens): one streaming pass over the logits.  It applies
//             the request processors (only to the tokens the history, bias and stop lists touch), finds the
//             chunk's best candidate, histograms the fixed-point weights by fine bin and writes the chunk's
//             record: exact per-power-of-two sums, the bin intervals the row's top-k / min-p / top-p
//             boundaries may fall in (one word per non-empty bin, with prefix sums, and the elements bucketed
//             by bin), and the processed values of the touched tokens.
//   k_resolve (B workgroups, one per row): merges the records, locates every boundary bin from exact
//             cumulative sums, resolves the boundary element inside that one bin, picks the chunk of the draw
//             by its exact kept mass and draws the token inside it (Philox4x32-10, inverse CDF in index order)
//             from one rescan of that chunk.  A boundary outside what the records cover sends the row to exact
//             rescans of its logits instead.
// The definition being computed is stated in oracle/sampler.py; the reference it restates is
// engine/src/proc.h:39-49 (processors), engine/src/mtp_sample.cu:122-183 (temperature / min_p / top-k /
// top-p), engine/src/mtp_sample.cu:10-27 (Philox draw) and engine/src/misc.cu:50-111 (argmax).
#include <math.h>
#include <stdlib.h>

#include "qws_device.h"

namespace qws {

constexpr int EPT = 8;                    // elements per thread of a chunk
constexpr int CH = NT * EPT;              // tokens per chunk
constexpr int TCAP = 1024;                // touched tokens per chunk processed sparsely (and handed over as patches)
constexpr int XN = 2048;                  // elements of one bin the resolver holds and sorts in LDS
constexpr int NBK = 2048;                 // buckets of the LDS sort
constexpr int MAXR = 4;                   // covered runs of bins the resolver tracks
constexpr int TOPB = 64;                  // top-p: every chunk hands over at least its best TOPB candidates
constexpr int MARGIN = 6;                 // top-p: fine bins on either side of the chunk's own nucleus boundary
constexpr int PP = (NBIN + NT - 1) / NT;  // fine bins per thread in block-wide bin scans

// ---------------------------------------------------------------------------------------------- chunk record
struct Head {
  uint32_t max_key, max_idx;     // best candidate (key, lowest index)
  int nexp;                      // floor(a) of the best: the chunk window is exponents [nexp - 38, nexp]
  int n_win;                     // candidates inside the window (0: none, or a greedy row)
  int n_el;                      // elements handed over, bucketed by bin (bins descending)
  int n_wd;                      // words: the non-empty bins of the intervals, descending
  int n_iv;                      // intervals (<= 2); interval 0 reaches the window top when top_set
  int top_set;
  int n_patch;                   // processed-value patches; > TCAP: none recorded (rebuild from the history)
  int pad0;
  int ivlo[MAXIV], ivhi[MAXIV];  // window-relative fine bins (0 = the window floor)
  uint32_t cnt_part[MAXIV];      // window interval: elements above ivhi inside ivhi's power of two
  uint64_t mu_part[MAXIV];       //                  their summed mantissas
  uint32_t ccnt[NEXP];           // per-power-of-two counts of the window (index 0 = the floor)
  uint32_t pad1;
  uint64_t cmu[NEXP];            // per-power-of-two summed mantissas
};
constexpr size_t HEAD_BYTES = (sizeof(Head) + 255) & ~(size_t)255;
constexpr size_t WORDS_OFF = HEAD_BYTES;                        // CAP words of 16 bytes
constexpr size_t ELEMS_OFF = WORDS_OFF + (size_t)CAP * 16;      // CAP elements: key << 32 | index
constexpr size_t PATCH_OFF = ELEMS_OFF + (size_t)CAP * 8;       // TCAP patches: local index << 32 | value bits
constexpr size_t REC_BYTES = PATCH_OFF + (size_t)TCAP * 8;

struct Layout {
  int G;                         // chunks per row
};
__device__ inline char* rec_of(char* ws, const Layout& L, int row, int g) { return ws + ((size_t)row * L.G + g) * REC_BYTES; }

// One non-empty bin of a chunk's intervals.  pc / pm: count and summed mantissas of this bin and of the interval's
// bins above it inside the same power of two.  Packed in 16 bytes:
//   w0 = bin | cnt << 12 | off << 23 | pc << 33 | mu[0:18) << 46,   w1 = pm | mu[18:37) << 37.
struct Word {
  int bin, cnt, off, pc;         // window-relative bin, elements, first element in the list, prefix count
  uint64_t pm, mu;               // prefix mantissa sum, the bin's own mantissa sum
};
constexpr uint64_t M37 = (1ull << 37) - 1;
__device__ inline void word_store(char* rec, int j, const Word& w) {
  uint64_t* p = (uint64_t*)(rec + WORDS_OFF) + 2 * j;
  p[0] = (uint64_t)w.bin | ((uint64_t)w.cnt << 12) | ((uint64_t)w.off << 23) | ((uint64_t)w.pc << 33) | ((w.mu & 0x3FFFFull) << 46);
  p[1] = w.pm | ((w.mu >> 18) << 37);
}
__device__ inline Word word_load(const char* rec, int j) {
  const uint4 v = *((const uint4*)(rec + WORDS_OFF) + j);
  const uint64_t w0 = ((uint64_t)v.y << 32) | v.x, w1 = ((uint64_t)v.w << 32) | v.z;
  Word w;
  w.bin = (int)(w0 & 0xFFF);
  w.cnt = (int)((w0 >> 12) & 0x7FF);
  w.off = (int)((w0 >> 23) & 0x3FF);
  w.pc = (int)((w0 >> 33) & 0x1FFF);
  w.pm = w1 & M37;
  w.mu = (w0 >> 46) | ((w1 >> 37) << 18);
  return w;
}

// ---------------------------------------------------------------------------------------------- chunk loading
template <int DT>
struct Vec { static constexpr int N = DT == QWS_DTYPE_F32 ? 4 : 8; };

// element e of this thread: index lo + (e / VEC * NT + tid) * VEC + e % VEC (increasing in e)
template <int DT>
__device__ inline int elt_index(int lo, int e) {
  constexpr int VEC = Vec<DT>::N;
  return lo + ((e / VEC) * NT + (int)threadIdx.x) * VEC + (e % VEC);
}

__device__ inline float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Raw logits of chunk [lo, hi) of a row: NaN -> -inf, -inf past hi.
template <int DT>
__device__ inline void load_raw(const qws_batch& B, int row, int lo, int hi, float (&x)[EPT]) {
  constexpr int VEC = Vec<DT>::N, S = EPT / VEC;
  const size_t esz = DT == QWS_DTYPE_F32 ? 4 : 2;
  const char* base = (const char*)B.logits + (size_t)row * (size_t)B.row_stride * esz;
#pragma unroll
  for (int s = 0; s < S; s++) {
    const int i0 = lo + (s * NT + (int)threadIdx.x) * VEC;
    if (i0 < hi) {
      if constexpr (DT == QWS_DTYPE_F32) {
        const float4 v = *(const float4*)(base + (size_t)i0 * 4);
        x[s * 4 + 0] = v.x;
        x[s * 4 + 1] = v.y;
        x[s * 4 + 2] = v.z;
        x[s * 4 + 3] = v.w;
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
  for (int e = 0; e < EPT; e++) x[e] = x[e] != x[e] ? -INFINITY : x[e];
}

// The banned / allowed bitmask: masked tokens become -inf (engine/src/proc.h:40).
template <int DT>
__device__ inline void apply_mask(const qws_batch& B, const qws_row& R, int lo, int hi, float (&x)[EPT]) {
  constexpr int VEC = Vec<DT>::N, S = EPT / VEC;
  if (!R.mask_mode) return;
  const unsigned* mrow = B.masks + (size_t)R.mask_row * (size_t)B.mask_words;
  const uint32_t flip = R.mask_mode == QWS_MASK_ALLOWED ? 0xFFFFFFFFu : 0u;
#pragma unroll
  for (int s = 0; s < S; s++) {
    const int i0 = lo + (s * NT + (int)threadIdx.x) * VEC;
    if (i0 >= hi) continue;
    const uint32_t mw = mrow[i0 >> 5] ^ flip;
#pragma unroll
    for (int j = 0; j < VEC; j++)
      if ((mw >> ((i0 + j) & 31)) & 1u) x[s * VEC + j] = -INFINITY;
  }
}

// Per-chunk processor state: tab[token - lo] = count | bias slot | stop | prompt (engine/src/proc.cu:72-103 builds
// the same state densely per request; here it is rebuilt per chunk from the row's history).  With tl, every token
// touched for the first time is appended to tl (up to TCAP) and counted in *nt.
__device__ inline void mark(uint32_t* tab, int j, uint32_t v, bool add, uint16_t* tl, int* nt) {
  const uint32_t old = add ? atomicAdd(&tab[j], v) : atomicOr(&tab[j], v);
  if (tl && old == 0u) {
    const int p = atomicAdd(nt, 1);
    if (p < TCAP) tl[p] = (uint16_t)j;
  }
}
__device__ void build_table(const qws_batch& B, const qws_row& R, int lo, int hi, uint32_t* tab, uint16_t* tl, int* nt) {
  for (int i = threadIdx.x; i < CH; i += NT) tab[i] = 0u;
  __syncthreads();
  const int* h = B.hist + R.hist_off;
  for (int j = threadIdx.x; j < R.n_prompt; j += NT) {
    const int id = h[j];
    if (id >= lo && id < hi) mark(tab, id - lo, TB_PROMPT, false, tl, nt);
  }
  for (int j = threadIdx.x; j < R.n_gen; j += NT) {
    const int id = h[R.n_prompt + j];
    if (id >= lo && id < hi) mark(tab, id - lo, 1u, true, tl, nt);
  }
  for (int j = threadIdx.x; j < R.n_drafts; j += NT) {
    const int id = B.drafts[R.draft_off + j];
    if (id >= lo && id < hi) mark(tab, id - lo, 1u, true, tl, nt);
  }
  if (R.min_tokens > R.ngen + R.n_drafts) {
    for (int j = threadIdx.x; j < R.n_stop; j += NT) {
      const int id = B.stop_ids[R.stop_off + j];
      if (id >= lo && id < hi) mark(tab, id - lo, TB_STOP, false, tl, nt);
    }
  }
  for (int j = threadIdx.x; j < R.n_bias; j += NT) {
    const int id = B.bias_ids[R.bias_off + j];
    if (id >= lo && id < hi) mark(tab, id - lo, (uint32_t)(j + 1) << TB_SLOT_SHIFT, false, tl, nt);
  }
  __syncthreads();
}

// engine/src/proc.h:41-48 on one (already masked) token, one IEEE rounding per operation
__device__ inline float proc_one(float x, uint32_t t, const qws_row& R, const float* bias_row) {
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

// x <-> a chunk-sized LDS array (index - lo)
template <int DT>
__device__ inline void stage(float* xs, float (&x)[EPT]) {
  constexpr int VEC = Vec<DT>::N, S = EPT / VEC;
#pragma unroll
  for (int s = 0; s < S; s++) {
    float4* p = (float4*)(xs + (s * NT + (int)threadIdx.x) * VEC);
#pragma unroll
    for (int q = 0; q < VEC / 4; q++) p[q] = make_float4(x[s * VEC + 4 * q], x[s * VEC + 4 * q + 1], x[s * VEC + 4 * q + 2], x[s * VEC + 4 * q + 3]);
  }
}
template <int DT>
__device__ inline void unstage(const float* xs, float (&x)[EPT]) {
  constexpr int VEC = Vec<DT>::N, S = EPT / VEC;
#pragma unroll
  for (int s = 0; s < S; s++) {
    const float4* p = (const float4*)(xs + (s * NT + (int)threadIdx.x) * VEC);
#pragma unroll
    for (int q = 0; q < VEC / 4; q++) {
      const float4 v = p[q];
      x[s * VEC + 4 * q] = v.x;
      x[s * VEC + 4 * q + 1] = v.y;
      x[s * VEC + 4 * q + 2] = v.z;
      x[s * VEC + 4 * q + 3] = v.w;
    }
  }
}

// ---------------------------------------------------------------------------------------------- block scans
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
__device__ inline uint64_t block_scan_u64(uint64_t v, uint64_t* red, uint64_t* total) {
  const int lane = lane_id(), w = wave_id();
  uint64_t s = v;
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t u = __shfl_up((unsigned long)s, o, 64);
    if (lane >= o) s += u;
  }
  __syncthreads();
  if (lane == 63) red[w] = s;
  __syncthreads();
  uint64_t before = 0, t = 0;
  for (int i = 0; i < NWAVE; i++) {
    if (i < w) before += red[i];
    t += red[i];
  }
  *total = t;
  return before + s;
}

// ---------------------------------------------------------------------------------------------- k_first
// hist word of a fine bin: (count << 40) | summed mantissas (< 2^36 for a chunk of 4,096 elements)
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

template <int DT>
__global__ void __launch_bounds__(NT) k_first(qws_batch B, Layout L, char* ws) {
  static_assert(NBIN * 8 >= CH * 4, "the staged chunk fits the histogram array");
  __shared__ __attribute__((aligned(16))) uint32_t tab[CH];               // processor table, then bin cursors
  __shared__ __attribute__((aligned(16))) unsigned long long hist[NBIN];  // staged chunk, then the histogram
  __shared__ float etab[256];
  __shared__ uint16_t tl[TCAP];
  __shared__ unsigned long long s_best;
  __shared__ uint64_t s_red[NWAVE];
  __shared__ uint64_t s_seg[MAXIV * NEXP];
  __shared__ int s_nt, s_niv;
  __shared__ int s_iv[2 * MAXIV];

  const int row = blockIdx.x / L.G, g = blockIdx.x - row * L.G;
  const int lo = g * CH, hi = min(B.V, lo + CH);
  const qws_row R = B.rows[row];
  char* rec = rec_of(ws, L, row, g);
  Head* H = (Head*)rec;
  float* xs = (float*)hist;

  float x[EPT];
  load_raw<DT>(B, row, lo, hi, x);
  if (threadIdx.x == 0) {
    s_best = 0ull;
    s_nt = 0;
  }
  if (threadIdx.x < 256) etab[threadIdx.x] = __uint_as_float(EXP2_TAB[threadIdx.x]);
  int nt = 0;
  if (R.proc_on) {
    apply_mask<DT>(B, R, lo, hi, x);
    build_table(B, R, lo, hi, tab, tl, &s_nt);
    nt = s_nt;
    const float* bias_row = B.bias_vals + R.bias_off;
    if (nt > TCAP) {  // dense: every token through the table
#pragma unroll
      for (int e = 0; e < EPT; e++) {
        const int i = elt_index<DT>(lo, e);
        if (i < hi) x[e] = proc_one(x[e], tab[i - lo], R, bias_row);
      }
    } else {
      // untouched tokens only get the zero bias (-0 + 0 = +0); the touched ones go through the staged copy
#pragma unroll
      for (int e = 0; e < EPT; e++) x[e] = x[e] + 0.0f;
      if (nt > 0) {
        stage<DT>(xs, x);
        __syncthreads();
        uint64_t* PT = (uint64_t*)(rec + PATCH_OFF);
        for (int p = threadIdx.x; p < nt; p += NT) {
          const int j = tl[p];
          const float v = proc_one(xs[j], tab[j], R, bias_row);
          xs[j] = v;
          PT[p] = ((uint64_t)j << 32) | __float_as_uint(v);
        }
        __syncthreads();
        unstage<DT>(xs, x);
      }
    }
  }
  if (B.out_logits) {
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const int i = elt_index<DT>(lo, e);
      if (i < hi) B.out_logits[(size_t)row * B.V + i] = x[e];
    }
  }
  // best candidate: a thread's elements come in increasing index, so the first of equal keys is kept
  uint32_t bk = 0, bi = 0;
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    const uint32_t k = okey(x[e]);
    if (k > bk) {
      bk = k;
      bi = (uint32_t)elt_index<DT>(lo, e);
    }
  }
  const uint64_t wb = wave_max_u64(comp(bk, bi));
  __syncthreads();  // the staged chunk is no longer read
  if (lane_id() == 0) atomicMax(&s_best, (unsigned long long)wb);
  for (int b = threadIdx.x; b < NBIN; b += NT) hist[b] = 0ull;
  __syncthreads();
  const uint64_t best = s_best;
  const uint32_t max_key = (uint32_t)(best >> 32), max_idx = 0xFFFFFFFFu - (uint32_t)best;
  if (!(R.temperature > 0.0f) || max_key == KEY_NEGINF) {
    if (threadIdx.x == 0) {
      H->max_key = max_key;
      H->max_idx = max_idx;
      H->nexp = 0;
      H->n_win = 0;
      H->n_el = 0;
      H->n_wd = 0;
      H->n_iv = 0;
      H->top_set = 0;
      H->n_patch = nt;
    }
    return;
  }
  const float kappa = kappa_f(R.temperature);
  const float amax = log2u(okey_val(max_key), kappa);
  const int Ng = weigh(amax, etab).n();
  const int base = (Ng - D_EXP) * FB;
  int rb[EPT];
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    const W w = weigh(log2u(x[e], kappa), etab);
    const int r = w.bin() - base;
    rb[e] = (x[e] != -INFINITY && r >= 0) ? r : -1;  // r < NBIN: the chunk's best lies in exponent Ng
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
  // ---- wave 0: the bins the resolver may need, as at most two intervals
  if (wave_id() == 0) {
    const int lane = lane_id();
    WaveView vw;
    vw.hist = hist;
    {  // per-exponent inclusive prefix from the top, lane u = exponent 38 - u
      uint32_t c = 0;
      float m = 0.0f;
      if (lane < NEXP) {
        const int e = D_EXP - lane;
        for (int b = 0; b < FB; b++) {  // lanes read distinct banks in turn
          const unsigned long long h = hist[e * FB + ((b + lane) & 63)];
          c += (uint32_t)(h >> HC_SHIFT);
          m += (float)(h & HM_MASK);
        }
        m = ldexpf(m, -lane - 23);
      }
      vw.cc = wave_scan_incl<uint32_t>(c);
      vw.cm = wave_scan_incl<float>(m);
    }
    const uint32_t ctot = vw.ccof(NEXP - 1);
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
        H->ivlo[0] = NBIN - 1 - floor_t;
        H->ivhi[0] = NBIN - 1;
        H->cnt_part[0] = 0;
        H->mu_part[0] = 0;
        s_iv[0] = NBIN - 1 - floor_t;
        s_iv[1] = NBIN - 1;
      }
      used = vw.cnt_to(floor_t);
      niv = 1;
    }
    if (topp && t_nuc > floor_t) {  // a window around the chunk's own top-p boundary
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
            H->ivlo[niv] = vlo;
            H->ivhi[niv] = vhi;
            H->cnt_part[niv] = (uint32_t)cp;
            H->mu_part[niv] = mp;
            s_iv[2 * niv] = vlo;
            s_iv[2 * niv + 1] = vhi;
          }
          niv++;
          break;
        }
      }
    }
    if (lane == 0) {
      H->max_key = max_key;
      H->max_idx = max_idx;
      H->nexp = Ng;
      H->n_win = (int)ctot;
      H->n_iv = niv;
      H->top_set = floor_t >= 0;
      H->n_patch = nt;
      s_niv = niv;
    }
  }
  __syncthreads();
  // ---- words: the non-empty bins of the intervals in descending order (interval 0 first), with prefix sums
  // inside each (interval, power of two) segment and the bins' element offsets.  Scan value of a position:
  // flag << 50 | count << 37 | summed mantissas.
  const int niv = s_niv;
  const int lo0 = niv > 0 ? s_iv[0] : 1, hi0 = niv > 0 ? s_iv[1] : 0;
  const int lo1 = niv > 1 ? s_iv[2] : 1, hi1 = niv > 1 ? s_iv[3] : 0;
  const int np0 = hi0 - lo0 + 1, np = np0 + (hi1 - lo1 + 1);
  uint64_t v[PP];
  uint64_t loc = 0;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int p = threadIdx.x * PP + k;
    v[k] = 0;
    if (p < np) {
      const int b = p < np0 ? hi0 - p : hi1 - (p - np0);
      const unsigned long long h = hist[b];
      const uint64_t c = h >> HC_SHIFT;
      if (c) v[k] = (1ull << 50) | (c << 37) | (h & HM_MASK);
    }
    loc += v[k];
  }
  uint64_t tot;
  const uint64_t incl = block_scan_u64(loc, s_red, &tot);
  uint64_t run = incl - loc;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int p = threadIdx.x * PP + k;
    if (p < np) {
      const int iv = p >= np0;
      const int b = iv ? hi1 - (p - np0) : hi0 - p;
      if (p == 0 || p == np0 || (b & 63) == 63) s_seg[iv * NEXP + (b >> 6)] = run;
    }
    run += v[k];
  }
  __syncthreads();
  run = incl - loc;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int p = threadIdx.x * PP + k;
    if (p < np && v[k]) {
      const int iv = p >= np0;
      const int b = iv ? hi1 - (p - np0) : hi0 - p;
      const uint64_t pre = run + v[k] - s_seg[iv * NEXP + (b >> 6)];
      Word w;
      w.bin = b;
      w.cnt = (int)((v[k] >> 37) & 0x1FFF);
      w.off = (int)((run >> 37) & 0x1FFF);
      w.pc = (int)((pre >> 37) & 0x1FFF);
      w.pm = pre & M37;
      w.mu = v[k] & M37;
      word_store(rec, (int)(run >> 50), w);
      tab[b] = (uint32_t)w.off;
    }
    run += v[k];
  }
  __syncthreads();
  // ---- elements of the intervals, bucketed by bin
  uint64_t* EL = (uint64_t*)(rec + ELEMS_OFF);
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    const int r = rb[e];
    if (r >= 0 && ((r >= lo0 && r <= hi0) || (r >= lo1 && r <= hi1))) {
      const uint32_t pos = atomicAdd(&tab[r], 1u);
      if (pos < (uint32_t)CAP) EL[pos] = ((uint64_t)okey(x[e]) << 32) | (uint64_t)(uint32_t)elt_index<DT>(lo, e);
    }
  }
  if (threadIdx.x == 0) {
    H->n_el = (int)((tot >> 37) & 0x1FFF);
    H->n_wd = (int)(tot >> 50);
  }
}

// ---------------------------------------------------------------------------------------------- resolver state
struct HS {                        // a chunk's head staged in LDS, plus per-row derived fields
  uint32_t max_key, max_idx;
  int nexp, n_win, n_el, n_wd, n_iv, top_set, n_patch;
  int ivlo[MAXIV], ivhi[MAXIV];
  uint32_t cnt_part[MAXIV];
  unsigned long long mu_part[MAXIV];
  int d;                           // row-relative bin of window-relative bin 0: (nexp - N) * 64
  int kr[MAXR];                    // interval holding covered run r (-1: none)
  int goff, gcnt, gpc;             // bin under resolution: its elements, and the word part of the sums above it
  unsigned long long gpm;
};
// interval of a chunk's bin: with a top set, interval 0 is the top set and 1 the window below it
__device__ inline int iv_of(const HS& h, int bin) { return h.top_set ? (bin >= h.ivlo[0] ? 0 : 1) : 0; }
// interval k in row-relative bins (the top set reaches the top of the row window)
__device__ inline void iv_row(const HS& h, int k, int* lo, int* hi) {
  *lo = h.ivlo[k] + h.d;
  *hi = (k == 0 && h.top_set) ? NBIN - 1 : h.ivhi[k] + h.d;
}

struct RowState {                  // per-row state of k_resolve (LDS)
  int G, V;
  uint32_t max_key, max_idx;
  float kappa, a_max, a_cut;       // a_cut: min_p keeps candidates with a >= a_cut
  int N;                           // exponent of the row's best: the row window is exponents [N - 38, N]
  int topk, minp, topp;
  u128 S_all;                      // window mass (units 2^(N - 38 - 23))
  unsigned long long n_win;
  int nrun;                        // covered runs, row-relative bins, descending
  int rlo[MAXR], rhi[MAXR];
  u128 am[MAXR];                   // exact mass / count above each run
  unsigned long long ac[MAXR];
};
struct Loc {
  int bin, run, ok;
  u128 cm;                         // exact mass before the bin (rank order)
  unsigned long long cc;           // count before the bin
};
struct Cut {
  uint64_t c;                      // comp of the last kept element
  u128 cm;                         // inclusive mass at it
  unsigned long long cc;           // inclusive count at it
  int ok;
};

// row histogram word of a fine bin: count << 45 | summed mantissas (< 2^42)
constexpr int HR_CSH = 45;
constexpr unsigned long long HR_MMASK = (1ull << HR_CSH) - 1;
constexpr int RT_BYTES = NBIN * 8 > CH * 4 ? NBIN * 8 : CH * 4;
constexpr int RX_BYTES = 2 * XN * 8;
static_assert(NBIN * 12 <= RX_BYTES && (NBIN + 1) * 4 <= RX_BYTES, "region X holds the rescan histogram");

struct Pool {                      // views of the resolver's LDS
  unsigned long long* hrow;        // region T: row histogram [NBIN]
  uint32_t* tab;                   // region T: processor table [CH] (rescans without patches)
  float* xs;                       // region T: staged chunk [CH]
  uint64_t *ea, *eb;               // region X: element buffers [XN]
  uint32_t* hc;                    // region X: rescan histogram counts [NBIN]
  unsigned long long* hm;          //           and summed mantissas [NBIN]
  int* cov;                        // region X: coverage differences [NBIN + 1]
  uint32_t *bcnt, *boff;           // sort buckets [NBK]
  uint8_t* cf;                     // covered flags [NBIN]
  float* etab;                     // exp2 table
  uint32_t* exc;                   // per-chunk power-of-two counts [MAXG][NEXP]
  unsigned long long* exm;         // per-chunk power-of-two summed mantissas [MAXG][NEXP]
  HS* hs;
  int* woff;                       // [MAXG + 1] first word of each chunk in the row's flat word order
  int* gbase;                      // [MAXG + 1] first gathered element of each chunk
  unsigned long long *mlo, *mhi;   // [MAXG] chunk kept masses (low / high halves)
  uint64_t* red64;
  u128* red128;
  uint32_t* redu;
  int* redi;
  int* si;
  u128* su;
  Loc* loc;
};

__device__ inline double u128_to_double(u128 v) { return (double)(uint64_t)(v >> 64) * 18446744073709551616.0 + (double)(uint64_t)v; }

// weight (units 2^(N - 38 - 23)) of a key; *mp = passes min_p
__device__ inline uint64_t key_weight(uint32_t key, const RowState& st, const float* etab, bool* mp) {
  const float a = log2u(okey_val(key), st.kappa);
  *mp = !st.minp || a >= st.a_cut;
  return wunits(weigh(a, etab), st.N);
}
// domain weight: > 0 only for candidates inside the row window that pass min_p
__device__ inline uint64_t dom_weight(uint32_t key, const RowState& st, const float* etab) {
  bool mp;
  const uint64_t w = key_weight(key, st, etab, &mp);
  return mp ? w : 0ull;
}

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

// ---------------------------------------------------------------------------------------------- chunk rescans
// The processed logits of chunk g exactly as k_first computed them: raw, mask, then the chunk's patches (or the
// processor table rebuilt from the history when k_first recorded none).  Uses region T.
template <int DT>
__device__ void load_processed(const qws_batch& B, const qws_row& R, int row, int g, const Layout& L, char* ws, const Pool& P, float (&x)[EPT]) {
  const int lo = g * CH, hi = min(B.V, lo + CH);
  load_raw<DT>(B, row, lo, hi, x);
  if (!R.proc_on) return;
  apply_mask<DT>(B, R, lo, hi, x);
  const float* bias_row = B.bias_vals + R.bias_off;
  const int n_patch = P.hs[g].n_patch;
  if (n_patch > TCAP) {
    build_table(B, R, lo, hi, P.tab, nullptr, nullptr);
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const int i = elt_index<DT>(lo, e);
      if (i < hi) x[e] = proc_one(x[e], P.tab[i - lo], R, bias_row);
    }
    __syncthreads();
    return;
  }
#pragma unroll
  for (int e = 0; e < EPT; e++) x[e] = x[e] + 0.0f;
  if (n_patch == 0) return;
  stage<DT>(P.xs, x);
  __syncthreads();
  const uint64_t* PT = (const uint64_t*)(rec_of(ws, L, row, g) + PATCH_OFF);
  for (int p = threadIdx.x; p < n_patch; p += NT) {
    const uint64_t v = PT[p];
    P.xs[(int)(v >> 32)] = __uint_as_float((uint32_t)v);
  }
  __syncthreads();
  unstage<DT>(P.xs, x);
  __syncthreads();
}

// Calls fn(index, x) for every finite processed logit of chunk g.
template <int DT, typename F>
__device__ inline void for_chunk(const qws_batch& B, const qws_row& R, int row, int g, const Layout& L, char* ws, const Pool& P, F fn) {
  const int lo = g * CH, hi = min(B.V, lo + CH);
  float x[EPT];
  load_processed<DT>(B, R, row, g, L, ws, P, x);
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    const int i = elt_index<DT>(lo, e);
    if (i < hi && x[e] != -INFINITY) fn(i, x[e]);
  }
  __syncthreads();
}

// Inverse CDF in index order inside chunk g over the kept set (domain weight > 0 and comp >= cut): the element
// whose kept-prefix interval contains t_local.  Returns the token or -1.
template <int DT>
__device__ int draw_in_chunk(const qws_batch& B, const qws_row& R, int row, int g, const Layout& L, char* ws, const RowState& st, uint64_t cut,
                             u128 t_local, const Pool& P) {
  constexpr int VEC = Vec<DT>::N, S = EPT / VEC;
  const int lo = g * CH, hi = min(st.V, lo + CH);
  float x[EPT];
  load_processed<DT>(B, R, row, g, L, ws, P, x);
  if (threadIdx.x == 0) P.si[7] = -1;
  __syncthreads();
  u128 run = 0;
#pragma unroll
  for (int s = 0; s < S; s++) {
    uint64_t w[VEC];
    u128 loc = 0;
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      const int e = s * VEC + j;
      const int i = elt_index<DT>(lo, e);
      w[j] = 0;
      if (i < hi && x[e] != -INFINITY) {
        const uint32_t k = okey(x[e]);
        if (comp(k, (uint32_t)i) >= cut) w[j] = dom_weight(k, st, P.etab);
      }
      loc += w[j];
    }
    u128 tot;
    const u128 inc = block_scan_u128(loc, P.red128, &tot);
    u128 c = run + inc - loc;
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      const u128 c2 = c + w[j];
      if (w[j] && c <= t_local && t_local < c2) P.si[7] = elt_index<DT>(lo, s * VEC + j);
      c = c2;
    }
    run += tot;
  }
  __syncthreads();
  const int tok = P.si[7];
  __syncthreads();
  return tok;
}

// Dense probabilities of the kept set (test-hook path).
template <int DT>
__device__ void write_probs(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, const RowState& st, uint64_t cut, u128 S2,
                            const Pool& P) {
  const double S2d = u128_to_double(S2);
  for (int g = 0; g < st.G; g++) {
    for_chunk<DT>(B, R, row, g, L, ws, P, [&](int i, float x) {
      const uint32_t k = okey(x);
      if (comp(k, (uint32_t)i) < cut) return;
      const uint64_t w = dom_weight(k, st, P.etab);
      if (w) B.out_probs[(size_t)row * st.V + i] = (float)((double)w / S2d);
    });
  }
}

// The chunk whose kept-mass interval (index order) contains t, from P.mlo / P.mhi; *tl = t minus the mass of the
// chunks before it.  -1: none.
__device__ int pick_chunk(u128 t, int G, const Pool& P, u128* tl) {
  if (wave_id() == 0) {
    const int lane = lane_id();
    const u128 m = lane < G ? (((u128)P.mhi[lane] << 64) | P.mlo[lane]) : (u128)0;
    u128 s = m;
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t lo = __shfl_up((unsigned long)(uint64_t)s, o, 64);
      const uint64_t hi = __shfl_up((unsigned long)(uint64_t)(s >> 64), o, 64);
      if (lane >= o) s += ((u128)hi << 64) | lo;
    }
    const bool hit = lane < G && m != 0 && t < s && t >= s - m;
    const unsigned long long bal = __ballot(hit);
    if (lane == 0) P.si[4] = bal ? __ffsll((long long)bal) - 1 : -1;
    if (hit) P.su[8] = t - (s - m);
  }
  __syncthreads();
  const int g = P.si[4];
  *tl = P.su[8];
  __syncthreads();
  return g;
}

// ---------------------------------------------------------------------------------------------- merge
// Stages the chunk heads and per-power-of-two sums, finds the row's best.  Returns 0 when the row is greedy or
// has no candidate (token written).
__device__ int merge_row(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, RowState& st, const Pool& P) {
  const int G = L.G;
  uint64_t best = 0;
  for (int g = threadIdx.x; g < G; g += NT) {
    const Head* H = (const Head*)rec_of(ws, L, row, g);
    HS h;
    h.max_key = H->max_key;
    h.max_idx = H->max_idx;
    h.nexp = H->nexp;
    h.n_win = H->n_win;
    h.n_el = H->n_el;
    h.n_wd = H->n_wd;
    h.n_iv = H->n_iv;
    h.top_set = H->top_set;
    h.n_patch = H->n_patch;
#pragma unroll
    for (int k = 0; k < MAXIV; k++) {
      h.ivlo[k] = H->ivlo[k];
      h.ivhi[k] = H->ivhi[k];
      h.cnt_part[k] = H->cnt_part[k];
      h.mu_part[k] = H->mu_part[k];
    }
    h.d = 0;
    P.hs[g] = h;
    const uint64_t c = comp(h.max_key, h.max_idx);
    best = c > best ? c : best;
  }
  best = block_max_u64(best, P.red64);
  const uint32_t max_key = (uint32_t)(best >> 32), max_idx = 0xFFFFFFFFu - (uint32_t)best;
  if (!(R.temperature > 0.0f) || max_key == KEY_NEGINF) {
    if (threadIdx.x == 0) {
      B.out_tokens[row] = (int)max_idx;
      if (B.out_info) B.out_info[row] = 2;
    }
    return 0;
  }
  if (threadIdx.x == 0) {
    st.G = G;
    st.V = B.V;
    st.max_key = max_key;
    st.max_idx = max_idx;
    st.kappa = kappa_f(R.temperature);
    st.a_max = log2u(okey_val(max_key), st.kappa);
    st.N = weigh(st.a_max, P.etab).n();
    st.topp = R.top_p < 1.0f;
    st.a_cut = (float)((double)st.a_max + R.log2_min_p);
    // min_p cuts into the row window only when a_cut lies above its floor
    st.minp = R.min_p > 0.0f && st.a_cut > (float)(st.N - D_EXP);
  }
  __syncthreads();
  const int N = st.N;
  u128 S = 0, n = 0;
  for (int p = threadIdx.x; p < G * NEXP; p += NT) {
    const int g = p / NEXP, e = p - g * NEXP;
    uint32_t c = 0;
    unsigned long long m = 0;
    if (P.hs[g].n_win) {
      const Head* H = (const Head*)rec_of(ws, L, row, g);
      c = H->ccnt[e];
      m = H->cmu[e];
    }
    P.exc[p] = c;
    P.exm[p] = m;
    const int sh = e + P.hs[g].nexp - N;
    if (sh >= 0) {
      S += (u128)m << sh;
      n += c;
    }
  }
  S = block_sum_u128(S, P.red128);
  n = block_sum_u128(n, P.red128);
  if (threadIdx.x == 0) {
    st.S_all = S;
    st.n_win = (unsigned long long)n;
    st.topk = R.top_k > 0 && (unsigned long long)R.top_k < (unsigned long long)n;
  }
  __syncthreads();
  return 1;
}

// ---------------------------------------------------------------------------------------------- covered runs
// Runs: maximal row bins that every chunk with window candidates hands over completely (its elements and
// words).  Inside a run the row histogram is exact; above each run the exact mass and count are known.
__device__ void find_runs(const Layout& L, RowState& st, const Pool& P) {
  const int G = L.G;
  int* cov = P.cov;
  for (int b = threadIdx.x; b <= NBIN; b += NT) cov[b] = 0;
  if (threadIdx.x == 0) P.si[0] = 0;
  __syncthreads();
  for (int g = threadIdx.x; g < G; g += NT) {
    HS& h = P.hs[g];
    h.d = (h.nexp - st.N) * FB;
    if (!h.n_win) continue;
    atomicAdd(&P.si[0], 1);
    for (int k = 0; k < h.n_iv; k++) {
      int a, b;
      iv_row(h, k, &a, &b);
      if (b < 0) continue;
      atomicAdd(&cov[max(a, 0)], 1);
      atomicSub(&cov[b + 1], 1);
    }
  }
  __syncthreads();
  const int nact = P.si[0];
  // coverage of bin b = -(sum of cov[b + 1 .. NBIN]): a top-down scan; thread t holds positions t * PP + k
  int c[PP];
  int lsum = 0;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k;
    if (t < NBIN) lsum += cov[NBIN - t];
    c[k] = lsum;
  }
  int tot;
  const int inc = block_scan_incl<int>(lsum, P.redi, &tot);
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k;
    if (t < NBIN) P.cf[NBIN - 1 - t] = nact > 0 && -(inc - lsum + c[k]) == nact;
  }
  __syncthreads();
  // run tops (covered, bin above not) numbered from the top
  int tf[PP];
  int lt = 0;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k, b = NBIN - 1 - t;
    tf[k] = t < NBIN && P.cf[b] && !(b + 1 < NBIN && P.cf[b + 1]);
    lt += tf[k];
  }
  int ntop;
  const int itop = block_scan_incl<int>(lt, P.redi, &ntop);
  int rr = itop - lt;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k, b = NBIN - 1 - t;
    if (t < NBIN && P.cf[b]) {
      rr += tf[k];
      const int r = rr - 1;
      if (r < MAXR) {
        if (tf[k]) st.rhi[r] = b;
        if (!(b > 0 && P.cf[b - 1])) st.rlo[r] = b;
      }
    }
  }
  if (threadIdx.x == 0) st.nrun = min(ntop, MAXR);
  __syncthreads();
  for (int p = threadIdx.x; p < G * MAXR; p += NT) {
    const int g = p / MAXR, r = p - g * MAXR;
    HS& h = P.hs[g];
    int kk = -1;
    if (r < st.nrun && h.n_win) {
      for (int k = 0; k < h.n_iv; k++) {
        int a, b;
        iv_row(h, k, &a, &b);
        if (a <= st.rlo[r] && st.rhi[r] <= b) kk = k;
      }
    }
    h.kr[r] = kk;
  }
  __syncthreads();
}

// Exact count and mass (row units) of chunk g's elements in powers of two above that of row bin b, plus, when
// b's power of two is that of the window interval's top, the elements above that top inside it.  Interval k of
// the chunk holds b.
__device__ inline void above_exps(const Pool& P, const HS& h, int g, int k, int b, int N, u128* m, unsigned long long* c) {
  const int E = (b - h.d) >> 6;      // b's power of two, window-relative
  const int sh0 = h.nexp - N;        // row shift of window-relative power 0
  u128 lm = 0;
  unsigned long long lc = 0;
  for (int e = E + 1; e < NEXP; e++) {
    lm += (u128)P.exm[g * NEXP + e] << (e + sh0);
    lc += P.exc[g * NEXP + e];
  }
  if (!(k == 0 && h.top_set) && (h.ivhi[k] >> 6) == E) {
    lm += (u128)h.mu_part[k] << (E + sh0);
    lc += h.cnt_part[k];
  }
  *m = lm;
  *c = lc;
}

// Flat loop over the row's words: fn(chunk, word index, word, next word's bin or -1).
template <typename F>
__device__ inline void for_words(char* ws, const Layout& L, int row, const Pool& P, F fn) {
  const int nw = P.woff[L.G];
  int g = 0;
  for (int i = threadIdx.x; i < nw; i += NT) {
    while (P.woff[g + 1] <= i) g++;
    const char* rec = rec_of(ws, L, row, g);
    const int j = i - P.woff[g];
    const Word w = word_load(rec, j);
    const int nb = j + 1 < P.hs[g].n_wd ? word_load(rec, j + 1).bin : -1;
    fn(g, j, w, nb);
  }
}
// word w (interval k of chunk h) is the lowest word above window-relative bin bc inside bc's power of two and
// interval: its prefix sums are the chunk's sums above bc inside that power of two
__device__ inline bool lowest_above(const HS& h, const Word& w, int k, int nb, int bc) {
  if ((w.bin >> 6) != (bc >> 6) || w.bin <= bc) return false;
  return !(nb >= 0 && iv_of(h, nb) == k && (nb >> 6) == (bc >> 6) && nb > bc);
}

// The row histogram of every handed-over bin and the exact mass / count above each run (st.am / st.ac).
__device__ void runs_above(char* ws, const Layout& L, int row, RowState& st, const Pool& P) {
  const int G = L.G, N = st.N, nrun = st.nrun;
  for (int b = threadIdx.x; b < NBIN; b += NT) P.hrow[b] = 0ull;
  const int nwd = threadIdx.x < G && P.hs[threadIdx.x].n_win ? P.hs[threadIdx.x].n_wd : 0;
  int tot;
  const int inc = block_scan_incl<int>(nwd, P.redi, &tot);
  if (threadIdx.x < G) P.woff[threadIdx.x] = inc - nwd;
  if (threadIdx.x == 0) P.woff[G] = tot;
  __syncthreads();
  u128 am[MAXR];
  unsigned long long ac[MAXR];
#pragma unroll
  for (int r = 0; r < MAXR; r++) {
    am[r] = 0;
    ac[r] = 0;
  }
  for_words(ws, L, row, P, [&](int g, int, const Word& w, int nb) {
    const HS& h = P.hs[g];
    const int rb = w.bin + h.d;
    if (rb >= 0) atomicAdd(&P.hrow[rb], ((unsigned long long)w.cnt << HR_CSH) | (unsigned long long)w.mu);
    const int k = iv_of(h, w.bin);
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
      if (r < nrun && h.kr[r] == k) {
        const int bc = st.rhi[r] - h.d;
        if (lowest_above(h, w, k, nb, bc)) {
          am[r] += (u128)w.pm << (st.rhi[r] >> 6);
          ac[r] += (unsigned long long)w.pc;
        }
      }
    }
  });
  for (int p = threadIdx.x; p < G * MAXR; p += NT) {
    const int g = p / MAXR, r = p - g * MAXR;
    const HS& h = P.hs[g];
    if (r >= nrun || h.kr[r] < 0) continue;
    u128 m;
    unsigned long long c;
    above_exps(P, h, g, h.kr[r], st.rhi[r], N, &m, &c);
#pragma unroll
    for (int q = 0; q < MAXR; q++)
      if (q == r) {
        am[q] += m;
        ac[q] += c;
      }
  }
#pragma unroll
  for (int r = 0; r < MAXR; r++) {
    const u128 m = block_sum_u128(am[r], P.red128);
    const u128 c = block_sum_u128((u128)ac[r], P.red128);
    if (threadIdx.x == 0 && r < nrun) {
      st.am[r] = m;
      st.ac[r] = (unsigned long long)c;
    }
  }
  __syncthreads();
}

// The covered bin where the cumulative (rank order) count (by_mass 0) / mass (1) first reaches target, or the
// covered row bin want (>= 0): with its exact cumulative mass and count before it.
__device__ Loc locate(const RowState& st, const Pool& P, int by_mass, u128 target, int want) {
  u128 vm[PP];
  unsigned long long vc[PP];
  int vr[PP];
  u128 lm = 0, lc = 0;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int t = threadIdx.x * PP + k, b = NBIN - 1 - t;
    vr[k] = -1;
    vm[k] = 0;
    vc[k] = 0;
    if (t < NBIN) {
      for (int r = 0; r < st.nrun; r++)
        if (st.rlo[r] <= b && b <= st.rhi[r]) vr[k] = r;
      if (vr[k] >= 0) {
        const unsigned long long h = P.hrow[b];
        vm[k] = (u128)(h & HR_MMASK) << (b >> 6);
        vc[k] = h >> HR_CSH;
      }
    }
    lm += vm[k];
    lc += vc[k];
  }
  u128 tm, tc;
  const u128 im = block_scan_u128(lm, P.red128, &tm);
  const u128 ic = block_scan_u128(lc, P.red128, &tc);
  if (threadIdx.x == 0) P.loc->ok = 0;
  u128 pm = im - lm, pc = ic - lc;
#pragma unroll
  for (int k = 0; k < PP; k++) {  // exclusive prefix at each run's top
    const int b = NBIN - 1 - (int)(threadIdx.x * PP + k);
    if (vr[k] >= 0 && b == st.rhi[vr[k]]) {
      P.su[2 * vr[k]] = pm;
      P.su[2 * vr[k] + 1] = pc;
    }
    pm += vm[k];
    pc += vc[k];
  }
  __syncthreads();
  pm = im - lm;
  pc = ic - lc;
#pragma unroll
  for (int k = 0; k < PP; k++) {
    const int b = NBIN - 1 - (int)(threadIdx.x * PP + k);
    if (vr[k] >= 0) {
      const int r = vr[k];
      const u128 bm = st.am[r] + pm - P.su[2 * r];
      const u128 bc = (u128)st.ac[r] + pc - P.su[2 * r + 1];
      const u128 before = by_mass ? bm : bc;
      const u128 after = before + (by_mass ? vm[k] : (u128)vc[k]);
      const bool hit = want >= 0 ? b == want : (before < target && after >= target);
      if (hit) {
        P.loc->bin = b;
        P.loc->run = r;
        P.loc->cm = bm;
        P.loc->cc = (unsigned long long)bc;
        P.loc->ok = 1;
      }
    }
    pm += vm[k];
    pc += vc[k];
  }
  __syncthreads();
  const Loc out = *P.loc;
  __syncthreads();
  return out;
}

// The elements of covered row bin b (in run rr) into P.ea, sorted in rank order, and per chunk the word part of
// the exact sums above b (h.gpc / h.gpm).  Returns their count, or -1 when they exceed XN.
__device__ int gather_bin(char* ws, const Layout& L, int row, int b, int rr, const Pool& P) {
  const int G = L.G;
  for (int g = threadIdx.x; g < G; g += NT) {
    HS& h = P.hs[g];
    h.goff = 0;
    h.gcnt = 0;
    h.gpc = 0;
    h.gpm = 0;
  }
  __syncthreads();
  for_words(ws, L, row, P, [&](int g, int, const Word& w, int nb) {
    HS& h = P.hs[g];
    const int k = iv_of(h, w.bin);
    if (h.kr[rr] != k) return;
    const int bc = b - h.d;
    if (w.bin == bc) {
      h.goff = w.off;
      h.gcnt = w.cnt;
    } else if (lowest_above(h, w, k, nb, bc)) {
      h.gpc = w.pc;
      h.gpm = w.pm;
    }
  });
  __syncthreads();
  const int c = threadIdx.x < G ? P.hs[threadIdx.x].gcnt : 0;
  int n;
  const int inc = block_scan_incl<int>(c, P.redi, &n);
  if (threadIdx.x < G) P.gbase[threadIdx.x] = inc - c;
  if (threadIdx.x == 0) P.gbase[G] = n;
  __syncthreads();
  if (n > XN) return -1;
  int g = 0;
  for (int i = threadIdx.x; i < n; i += NT) {
    while (P.gbase[g + 1] <= i) g++;
    const uint64_t v = ((const uint64_t*)(rec_of(ws, L, row, g) + ELEMS_OFF))[P.hs[g].goff + i - P.gbase[g]];
    P.ea[i] = comp((uint32_t)(v >> 32), (uint32_t)v);
  }
  __syncthreads();
  if (n > 1) lds_sort_desc(P.ea, P.eb, n, P);
  return n;
}

// Inside a gathered bin (P.ea[0, n), rank order): the first element whose inclusive cumulative count
// (by_mass 0) or mass (1) reaches target, starting from (cm, cc) before the bin; elements outside the domain
// weigh and count 0.  by_mass 2: the bin's totals.
__device__ Cut walk(int n, const RowState& st, const Pool& P, u128 cm, unsigned long long cc, int by_mass, u128 target) {
  Cut out = {0, 0, 0, 0};
  const int Q = (n + NT - 1) / NT;
  const int j0 = min(n, (int)threadIdx.x * Q), j1 = min(n, j0 + Q);
  u128 lm = 0, lc = 0;
  for (int j = j0; j < j1; j++) {
    const uint64_t wt = dom_weight((uint32_t)(P.ea[j] >> 32), st, P.etab);
    lm += wt;
    lc += wt ? 1 : 0;
  }
  u128 tm, tc;
  const u128 im = block_scan_u128(lm, P.red128, &tm);
  const u128 ic = block_scan_u128(lc, P.red128, &tc);
  if (by_mass == 2) {
    out.cm = cm + tm;
    out.cc = cc + (unsigned long long)tc;
    out.ok = 1;
    return out;
  }
  if (threadIdx.x == 0) P.si[2] = -1;
  __syncthreads();
  u128 m = cm + im - lm, c = (u128)cc + ic - lc;
  for (int j = j0; j < j1; j++) {
    const uint64_t wt = dom_weight((uint32_t)(P.ea[j] >> 32), st, P.etab);
    const u128 m2 = m + wt, c2 = c + (wt ? 1 : 0);
    const u128 before = by_mass ? m : c, after = by_mass ? m2 : c2;
    if (wt && before < target && after >= target) {
      P.si[2] = j;
      P.su[10] = m2;
      P.su[11] = c2;
    }
    m = m2;
    c = c2;
  }
  __syncthreads();
  const int js = P.si[2];
  if (js >= 0) {
    out.c = P.ea[js];
    out.cm = P.su[10];
    out.cc = (unsigned long long)P.su[11];
    out.ok = 1;
  }
  __syncthreads();
  return out;
}

// Kept mass of every chunk (comp >= cut, in the domain) with the boundary in covered row bin b of run rr; P.ea[0, n)
// holds bin b's elements and h.gpm the word parts (gather_bin of b).  -> P.mlo / P.mhi
__device__ void chunk_masses(int n, int b, int rr, uint64_t cut, const RowState& st, const Pool& P) {
  for (int g = threadIdx.x; g < st.G; g += NT) {
    const HS& h = P.hs[g];
    u128 m = 0;
    if (h.n_win && h.kr[rr] >= 0) {
      unsigned long long c;
      above_exps(P, h, g, h.kr[rr], b, st.N, &m, &c);
      m += (u128)h.gpm << (b >> 6);
    }
    P.mlo[g] = (unsigned long long)m;
    P.mhi[g] = (unsigned long long)(m >> 64);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += NT) {
    const uint64_t v = P.ea[i];
    if (v < cut) continue;
    const uint64_t w = dom_weight((uint32_t)(v >> 32), st, P.etab);
    if (!w) continue;
    const int g = (int)((0xFFFFFFFFu - (uint32_t)v) / (uint32_t)CH);
    const unsigned long long old = atomicAdd(&P.mlo[g], (unsigned long long)w);
    if (old + w < old) atomicAdd(&P.mhi[g], 1ull);
  }
  __syncthreads();
}

// Resolves a row from the chunk records.  Returns 1 when the token is written, 0 when a boundary lies outside the
// covered bins (the caller then rescans).
template <int DT>
__device__ int resolve_records(const qws_batch& B, const qws_row& Rw, int row, const Layout& L, char* ws, RowState& st, const Pool& P, uint32_t u24) {
  find_runs(L, st, P);
  if (st.nrun == 0) return 0;
  runs_above(ws, L, row, st, P);
  // ---- min_p: the domain ends inside the bin of a_cut
  bool minp = st.minp;
  int bm = -1, bm_run = -1, n = 0;
  u128 Dm = st.S_all;
  unsigned long long Dc = st.n_win;
  if (minp) {
    bm = weigh(st.a_cut, P.etab).bin() - (st.N - D_EXP) * FB;
    if (bm < 0) {
      minp = false;
    } else {
      const Loc lb = locate(st, P, 1, 0, bm);
      if (!lb.ok) return 0;
      n = gather_bin(ws, L, row, bm, lb.run, P);
      if (n < 0) return 0;
      const Cut t = walk(n, st, P, lb.cm, lb.cc, 2, 0);
      Dm = t.cm;
      Dc = t.cc;
      bm_run = lb.run;
    }
  }
  // ---- top-k
  int bin_c = -1, run_c = -1;
  uint64_t cut = 0;
  u128 S = Dm;
  if (Rw.top_k > 0 && (unsigned long long)Rw.top_k < Dc) {
    const Loc lk = locate(st, P, 0, (u128)Rw.top_k, -1);
    if (!lk.ok) return 0;
    n = gather_bin(ws, L, row, lk.bin, lk.run, P);
    if (n < 0) return 0;
    const Cut ck = walk(n, st, P, lk.cm, lk.cc, 0, (u128)Rw.top_k);
    if (!ck.ok) return 0;
    bin_c = lk.bin;
    run_c = lk.run;
    cut = ck.c;
    S = ck.cm;
  }
  // ---- top-p
  if (st.topp) {
    const u128 TP = (u128)(uint64_t)floor((double)Rw.top_p * 4294967296.0);
    u128 thr = (TP * S + (((u128)1 << 32) - 1)) >> 32;
    if (thr == 0) thr = 1;  // the first candidate: every inclusive sum reaches 0 (and 1)
    const Loc lp = locate(st, P, 1, thr, -1);
    if (!lp.ok) return 0;
    n = gather_bin(ws, L, row, lp.bin, lp.run, P);
    if (n < 0) return 0;
    const Cut cp = walk(n, st, P, lp.cm, lp.cc, 1, thr);
    if (!cp.ok) return 0;
    bin_c = lp.bin;
    run_c = lp.run;
    cut = cp.c;
    S = cp.cm;
  }
  if (bin_c < 0) {
    if (!minp) return 0;
    bin_c = bm;  // min_p alone: bin bm was gathered last
    run_c = bm_run;
    cut = 0;
  }
  // ---- draw: chunk by kept mass, then inside the chunk
  chunk_masses(n, bin_c, run_c, cut, st, P);
  const u128 t = ((u128)u24 * S) >> 24;
  u128 tl;
  const int g = pick_chunk(t, L.G, P, &tl);
  if (g < 0) return 0;
  const int tok = draw_in_chunk<DT>(B, Rw, row, g, L, ws, st, cut, tl, P);
  if (tok < 0) return 0;
  if (B.out_probs) write_probs<DT>(B, Rw, row, L, ws, st, cut, S, P);
  if (threadIdx.x == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = 0;
  }
  return 1;
}

// No selection: every window candidate is kept; the chunk masses are exact from the power-of-two sums.
template <int DT>
__device__ void draw_pure(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, const RowState& st, const Pool& P, uint32_t u24) {
  for (int g = threadIdx.x; g < st.G; g += NT) {
    const HS& h = P.hs[g];
    u128 m = 0;
    if (h.n_win) {
      for (int e = 0; e < NEXP; e++) {
        const int sh = e + h.nexp - st.N;
        if (sh >= 0) m += (u128)P.exm[g * NEXP + e] << sh;
      }
    }
    P.mlo[g] = (unsigned long long)m;
    P.mhi[g] = (unsigned long long)(m >> 64);
  }
  __syncthreads();
  const u128 t = ((u128)u24 * st.S_all) >> 24;
  u128 tl;
  const int g = pick_chunk(t, L.G, P, &tl);
  const int tok = g < 0 ? -1 : draw_in_chunk<DT>(B, R, row, g, L, ws, st, 0, tl, P);
  if (B.out_probs) write_probs<DT>(B, R, row, L, ws, st, 0, st.S_all, P);
  if (threadIdx.x == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = 3;
  }
}

// ---------------------------------------------------------------------------------------------- rescan fallback
struct Sel {
  uint64_t c;       // comp of the selected element
  u128 cnt, mass;   // inclusive cumulative count / mass at it
  int ok;
};

// Exact selection by rescans: the first domain element in comp order (descending) whose inclusive cumulative
// count (by_mass 0) or mass (1) reaches target.
template <int DT>
__device__ Sel select_rescan(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, const RowState& st, int by_mass, u128 target,
                             const Pool& P) {
  Sel out = {0, 0, 0, 0};
  const long long wbase = ((long long)st.N - D_EXP) * FB;
  // ---- level 1: histogram over the weight window's bins
  for (int b = threadIdx.x; b < NBIN; b += NT) {
    P.hc[b] = 0u;
    P.hm[b] = 0ull;
  }
  __syncthreads();
  for (int g = 0; g < st.G; g++) {
    for_chunk<DT>(B, R, row, g, L, ws, P, [&](int, float x) {
      const float a = log2u(x, st.kappa);
      if (st.minp && !(a >= st.a_cut)) return;
      const W w = weigh(a, P.etab);
      const long long rb = (long long)w.bin() - wbase;
      if (rb < 0) return;
      atomicAdd(&P.hc[rb], 1u);
      atomicAdd(&P.hm[rb], (unsigned long long)w.mu);
    });
  }
  // top-down scan: thread j owns top-down positions [j * PP, j * PP + PP)
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
  const u128 pm = im - lm, pc = ic - lc;
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
      P.red64[0] = ~0ull;  // running min / max of the set (red64 is free between block reductions)
      P.red64[1] = 0ull;
    }
    __syncthreads();
    for (int g = 0; g < st.G; g++) {
      for_chunk<DT>(B, R, row, g, L, ws, P, [&](int i, float x) {
        const float a = log2u(x, st.kappa);
        if (st.minp && !(a >= st.a_cut)) return;
        const W w = weigh(a, P.etab);
        if ((long long)w.bin() != bin_abs) return;
        const uint64_t c = comp(okey(x), (uint32_t)i);
        if (c < cmin || c > cmax) return;
        const int pos = atomicAdd(&P.si[1], 1);
        if (pos < XN) P.ea[pos] = c;
        atomicMin((unsigned long long*)&P.red64[0], (unsigned long long)c);
        atomicMax((unsigned long long*)&P.red64[1], (unsigned long long)c);
      });
    }
    const int n = P.si[1];
    cmin = P.red64[0];
    cmax = P.red64[1];
    __syncthreads();
    if (n <= XN) {
      if (n > 1) lds_sort_desc(P.ea, P.eb, n, P);
      const int Q = (n + NT - 1) / NT;
      const int j0 = min(n, (int)threadIdx.x * Q), j1 = min(n, j0 + Q);
      u128 loc = 0;
      for (int j = j0; j < j1; j++) loc += by_mass ? (u128)dom_weight((uint32_t)(P.ea[j] >> 32), st, P.etab) : (u128)1;
      u128 tot;
      const u128 inc = block_scan_u128(loc, P.red128, &tot);
      u128 cum = (by_mass ? mass_above : cnt_above) + inc - loc;
      if (threadIdx.x == 0) P.si[2] = -1;
      __syncthreads();
      for (int j = j0; j < j1; j++) {
        const u128 c2 = cum + (by_mass ? (u128)dom_weight((uint32_t)(P.ea[j] >> 32), st, P.etab) : (u128)1);
        if (cum < target && c2 >= target) P.si[2] = j;
        cum = c2;
      }
      __syncthreads();
      const int js = P.si[2];
      if (js < 0) return out;
      u128 lmass = 0, lcnt = 0;
      for (int j = j0; j < min(j1, js + 1); j++) {
        lmass += dom_weight((uint32_t)(P.ea[j] >> 32), st, P.etab);
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
    unsigned long long* dm = (unsigned long long*)P.eb;  // NBK mantissa sums
    for (int d = threadIdx.x; d < NBK; d += NT) {
      dc[d] = 0u;
      dm[d] = 0ull;
    }
    __syncthreads();
    for (int g = 0; g < st.G; g++) {
      for_chunk<DT>(B, R, row, g, L, ws, P, [&](int i, float x) {
        const float a = log2u(x, st.kappa);
        if (st.minp && !(a >= st.a_cut)) return;
        const W w = weigh(a, P.etab);
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

// Kept mass of chunk g (domain weight, comp >= cut) by a rescan.
template <int DT>
__device__ u128 chunk_mass(const qws_batch& B, const qws_row& R, int row, int g, const Layout& L, char* ws, const RowState& st, uint64_t cut,
                           const Pool& P) {
  u128 loc = 0;
  for_chunk<DT>(B, R, row, g, L, ws, P, [&](int i, float x) {
    const uint32_t k = okey(x);
    if (comp(k, (uint32_t)i) >= cut) loc += dom_weight(k, st, P.etab);
  });
  return block_sum_u128(loc, P.red128);
}

// The whole row by exact rescans of its logits (boundaries outside the records' covered bins).
template <int DT>
__device__ __attribute__((noinline)) void resolve_rescan(const qws_batch& B, const qws_row& R, int row, const Layout& L, char* ws, const RowState& st,
                                                         const Pool& P, uint32_t u24) {
  uint64_t cut = 0;
  u128 S = st.S_all;
  bool ok = true;
  if (st.minp) {
    u128 loc = 0;
    for (int g = 0; g < st.G; g++)
      for_chunk<DT>(B, R, row, g, L, ws, P, [&](int, float x) { loc += dom_weight(okey(x), st, P.etab); });
    S = block_sum_u128(loc, P.red128);
  }
  if (st.topk) {
    const Sel s = select_rescan<DT>(B, R, row, L, ws, st, 0, (u128)R.top_k, P);
    if (s.ok) {
      cut = s.c;
      S = s.mass;
    }  // else: fewer than K domain elements: top-k keeps them all
  }
  if (st.topp) {
    const u128 TP = (u128)(uint64_t)floor((double)R.top_p * 4294967296.0);
    u128 thr = (TP * S + (((u128)1 << 32) - 1)) >> 32;
    if (thr == 0) thr = 1;
    const Sel s = select_rescan<DT>(B, R, row, L, ws, st, 1, thr, P);
    if (s.ok) {
      cut = s.c;
      S = s.mass;
    } else {
      ok = false;
    }
  }
  int tok = -1;
  if (ok) {
    for (int g = 0; g < st.G; g++) {
      const u128 m = chunk_mass<DT>(B, R, row, g, L, ws, st, cut, P);
      if (threadIdx.x == 0) {
        P.mlo[g] = (unsigned long long)m;
        P.mhi[g] = (unsigned long long)(m >> 64);
      }
    }
    __syncthreads();
    const u128 t = ((u128)u24 * S) >> 24;
    u128 tl;
    const int g = pick_chunk(t, st.G, P, &tl);
    if (g >= 0) tok = draw_in_chunk<DT>(B, R, row, g, L, ws, st, cut, tl, P);
    if (B.out_probs) write_probs<DT>(B, R, row, L, ws, st, cut, S, P);
  }
  if (threadIdx.x == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = ok ? 1 : -1;
  }
}

// ---------------------------------------------------------------------------------------------- k_resolve
template <int DT>
__global__ void __launch_bounds__(NT) k_resolve(qws_batch B, Layout L, char* ws) {
  __shared__ __attribute__((aligned(16))) unsigned char regT[RT_BYTES];
  __shared__ __attribute__((aligned(16))) unsigned char regX[RX_BYTES];
  __shared__ __attribute__((aligned(16))) uint32_t regK[2 * NBK];
  __shared__ float etab[256];
  __shared__ uint32_t exc[MAXG * NEXP];
  __shared__ unsigned long long exm[MAXG * NEXP];
  __shared__ HS hs[MAXG];
  __shared__ int woff[MAXG + 1], gbase[MAXG + 1];
  __shared__ unsigned long long mlo[MAXG], mhi[MAXG];
  __shared__ uint8_t cf[NBIN];
  __shared__ uint64_t red64[NWAVE];
  __shared__ u128 red128[NWAVE];
  __shared__ uint32_t redu[NWAVE];
  __shared__ int redi[NWAVE];
  __shared__ int si[8];
  __shared__ u128 su[12];
  __shared__ Loc sloc;
  __shared__ RowState st;
  Pool P;
  P.hrow = (unsigned long long*)regT;
  P.tab = (uint32_t*)regT;
  P.xs = (float*)regT;
  P.ea = (uint64_t*)regX;
  P.eb = P.ea + XN;
  P.hc = (uint32_t*)regX;
  P.hm = (unsigned long long*)(regX + ((NBIN * 4 + 15) & ~15));
  P.cov = (int*)regX;
  P.bcnt = regK;
  P.boff = regK + NBK;
  P.cf = cf;
  P.etab = etab;
  P.exc = exc;
  P.exm = exm;
  P.hs = hs;
  P.woff = woff;
  P.gbase = gbase;
  P.mlo = mlo;
  P.mhi = mhi;
  P.red64 = red64;
  P.red128 = red128;
  P.redu = redu;
  P.redi = redi;
  P.si = si;
  P.su = su;
  P.loc = &sloc;
  if (threadIdx.x < 256) etab[threadIdx.x] = __uint_as_float(EXP2_TAB[threadIdx.x]);
  const int row = blockIdx.x;
  const qws_row R = B.rows[row];
  if (!merge_row(B, R, row, L, ws, st, P)) return;
  const uint32_t u24 = draw_u24(R.seed, R.position, R.stream, R.row_key, 0);
  if (!(st.topk || st.minp || st.topp)) {
    draw_pure<DT>(B, R, row, L, ws, st, P, u24);
    return;
  }
  if (resolve_records<DT>(B, R, row, L, ws, st, P, u24)) return;
  __syncthreads();
  resolve_rescan<DT>(B, R, row, L, ws, st, P, u24);
}

}  // namespace qws

// ---------------------------------------------------------------------------------------------- launcher
namespace qws {
static Layout layout_for(int V) {
  Layout L;
  L.G = (V + CH - 1) / CH;
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

template <int DT>
static hipError_t launch(const qws_batch& b, const Layout& L, char* ws, hipStream_t st) {
  const bool tm = g_timing.on && g_timing.n < Timing::CAPN;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][0], st);
  hipLaunchKernelGGL((k_first<DT>), dim3(b.B * L.G), dim3(NT), 0, st, b, L, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][1], st);
  hipLaunchKernelGGL((k_resolve<DT>), dim3(b.B), dim3(NT), 0, st, b, L, ws);
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
  const qws::Layout L = qws::layout_for(V);
  return (size_t)B * L.G * qws::REC_BYTES;
}

extern "C" int qws_sample(const qws_batch* b, void* ws, size_t ws_bytes, void* stream) {
  using namespace qws;
  if (!b || !b->logits || !b->rows || !b->out_tokens || !ws) return QWS_ERR_INVALID;
  if (b->B < 1 || b->V < 8 || (b->V & 7) || (b->row_stride & 7) || b->row_stride < 0) return QWS_ERR_INVALID;
  if (b->row_stride != 0 && b->row_stride < b->V) return QWS_ERR_INVALID;
  if (b->dtype != QWS_DTYPE_F32 && b->dtype != QWS_DTYPE_BF16) return QWS_ERR_INVALID;
  if (((uintptr_t)b->logits & 15) || ((uintptr_t)ws & 255)) return QWS_ERR_INVALID;
  if (b->masks && b->mask_words * 32LL < b->V) return QWS_ERR_INVALID;
  const Layout L = layout_for(b->V);
  if (L.G > MAXG) return QWS_ERR_NOT_SUPPORTED;
  if (ws_bytes < (size_t)b->B * L.G * REC_BYTES) return QWS_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  char* w = (char*)ws;
  const hipError_t e = b->dtype == QWS_DTYPE_F32 ? launch<QWS_DTYPE_F32>(*b, L, w, st) : launch<QWS_DTYPE_BF16>(*b, L, w, st);
  return (int)e;
}
