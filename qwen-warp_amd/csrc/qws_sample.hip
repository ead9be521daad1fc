// qws sampling kernels for MI355X (gfx950).
//
// One call samples B rows of V logits in two launches:
//   k_scan    (B x G workgroups, one per block of 8,192 tokens): one streaming pass over the logits.  It applies the
//             request processors, finds the block's best candidate and builds an exact LDS histogram of the
//             fixed-point weights by fine bin (a = x / T in log2 units, 64 bins per power of two).  Its record holds
//             the exact per-power-of-two sums (the row's total mass and the mass above any power of two follow by
//             realignment) and one window of bins, chosen from the block's own exact data, whose elements it lists
//             bucketed by bin: the block's whole top set when that is small (top-k, min-p, peaked top-p rows), or
//             the bins around the block's own top-p boundary (flat rows).
//   k_resolve (B workgroups, one per row): merges the records into row-level cumulative masses and counts that are
//             exact wherever every block's record pins them, locates the min-p, top-k and top-p boundaries, resolves
//             each inside its one fine bin from the listed elements, picks the block of the draw by its exact kept
//             mass and draws the token inside it (Philox4x32-10, inverse CDF in index order) from one rescan of that
//             block.  A boundary the records do not pin sends the row to exact rescans of its logits instead.
// The definition being computed is stated in oracle/sampler.py; the reference it restates is
// engine/src/proc.h:39-49 (processors), engine/src/mtp_sample.cu:122-183 (temperature / min_p / top-k /
// top-p), engine/src/mtp_sample.cu:10-27 (Philox draw) and engine/src/misc.cu:50-111 (argmax).
#include <math.h>
#include <stdlib.h>

#include "qws_block.h"

namespace qws {

constexpr int NT1 = 512, NWV1 = NT1 / 64;    // k_scan workgroup
constexpr int NT2 = 1024, NWV2 = NT2 / 64;   // k_resolve workgroup
constexpr int CAP = 1024;                    // elements a block may list
constexpr int MARGIN = 6;                    // top-p: fine bins listed on either side of the block's own boundary
constexpr int MAXG = 64;                     // blocks per row (V <= 524,288)
constexpr int NR = NBIN;                     // row bins with a nonzero weight (row-relative, 0 = the top)
constexpr int XN = 2048;                     // elements of one bin k_resolve holds in LDS
constexpr unsigned long long M40 = (1ull << 40) - 1;

// ---------------------------------------------------------------------------------------------- block record
enum : int { RF_CAND = 1, RF_SAMP = 2, RF_WIN = 4, RF_OVER = 8 };
// Bins of a block are top-down: rel = (c * 64 + 63) - fine bin, so rel 0..63 is the power of two 2^c of the block's
// best and rel >> 6 = e counts powers of two below it.  Elements with rel >= NBIN weigh nothing in any row window.
struct Rec {
  uint32_t max_key, max_idx;     // best candidate (okey, lowest index); KEY_NEGINF: none
  int c, flags;                  // power of two of the best; RF_*
  int rel_max, rel_min;          // bins of the best and of the lowest candidate with rel < NBIN
  int w0, w1;                    // listed window, rel w0..w1 (w0 <= w1 with RF_WIN)
  uint32_t n_pos, n_win;         // candidates with rel < NBIN; listed elements
  uint32_t pcnt, pad;            // elements of power of two w0 >> 6 above w0
  unsigned long long pmu;        // their summed mantissas
  uint32_t ecnt[NEXP];           // per power of two e (rel >> 6): candidates
  unsigned long long emu[NEXP];  //                                  summed mantissas
};
constexpr size_t HDR_BYTES = 512;
static_assert(sizeof(Rec) <= HDR_BYTES, "record header");
constexpr size_t REC_BYTES = HDR_BYTES + (size_t)CAP * 8;   // then CAP elements: comp(key, index), bucketed by bin
__device__ inline char* rec_of(char* ws, int G, int row, int g) { return ws + ((size_t)row * G + g) * REC_BYTES; }

// ---------------------------------------------------------------------------------------------- k_scan
template <int DT>
__global__ void __launch_bounds__(NT1) k_scan(qws_batch B, int G, char* ws) {
  using BL = Blk<DT, NT1>;
  constexpr int EPT = BL::EPT;
  constexpr int PP = (NBIN + NT1 - 1) / NT1;
  __shared__ __attribute__((aligned(16))) uint32_t s_tab[BLK];   // processor table, then histogram / cursors
  __shared__ __attribute__((aligned(16))) float2 s_ts[1024];
  __shared__ uint32_t s_ecnt[NEXP];
  __shared__ unsigned long long s_emu[NEXP];
  __shared__ float s_redf[NWV1];
  __shared__ uint32_t s_redu[NWV1];
  __shared__ uint32_t s_imin;
  __shared__ int s_win[8];
  __shared__ unsigned long long s_pm;

  const int row = blockIdx.x / G, g = blockIdx.x - row * G;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  const qws_row R = B.rows[row];
  char* rec = rec_of(ws, G, row, g);
  Rec* H = (Rec*)rec;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();

  float x[EPT];
  load_processed<DT, NT1>(B, R, row, lo, hi, s_tab, x);
  if (B.out_logits) {
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const int i = lo + BL::local(e);
      if (i < hi) B.out_logits[(size_t)row * B.V + i] = x[e];
    }
  }
  // ---- best candidate: the largest value, lowest index
  float mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < EPT; e++) mloc = fmaxf(mloc, x[e]);
  const float mw = wave_max_f(mloc);
  if (lane == 0) s_redf[wave] = mw;
  if (tid == 0) s_imin = 0xFFFFFFFFu;
  __syncthreads();
  float M = s_redf[0];
  for (int i = 1; i < NWV1; i++) M = fmaxf(M, s_redf[i]);
  if (M != -INFINITY && mloc == M) {  // equal values compare equal across -0 / +0
    uint32_t im = 0xFFFFFFFFu;
#pragma unroll
    for (int e = EPT - 1; e >= 0; e--)
      if (x[e] == M) im = (uint32_t)(lo + BL::local(e));
    atomicMin(&s_imin, im);
  }
  const float K = kscale(R.temperature);
  const bool samp = R.temperature > 0.0f && K < INFINITY;
  __syncthreads();
  const uint32_t imax = s_imin;
  if (M == -INFINITY || !samp) {
    if (tid == 0) {
      H->max_key = M == -INFINITY ? KEY_NEGINF : okey(M);
      H->max_idx = M == -INFINITY ? 0u : imax;
      H->flags = M == -INFINITY ? 0 : RF_CAND;
      H->n_pos = 0;
      H->n_win = 0;
    }
    return;
  }
  // ---- exact histogram of the weights by fine bin, top-down from the best's power of two
  ((uint4*)s_ts)[tid] = ((const uint4*)EXP2_TS)[tid];
  const W wm = weigh(tval(M, K), ts_const());
  const int c = wm.n();
  const int btop = c * FB + (FB - 1);
  unsigned long long* hist = (unsigned long long*)s_tab;
  for (int i = tid; i < NBIN; i += NT1) hist[i] = 0ull;
  __syncthreads();
  uint32_t rp[EPT / 2];  // the elements' bins (16 bits each; 0xFFFF: not in the window)
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    uint32_t rel = 0xFFFFu;
    if (x[e] != -INFINITY) {
      const W w = weigh(tval(x[e], K), s_ts);
      const int r = btop - w.bin();
      if (r < NBIN) {
        atomicAdd(&hist[r], (1ull << 40) | (unsigned long long)w.mu);
        rel = (uint32_t)r;
      }
    }
    if (e & 1)
      rp[e >> 1] |= rel << 16;
    else
      rp[e >> 1] = rel;
  }
  __syncthreads();
  for (int u = wave; u < NEXP; u += NWV1) {
    const unsigned long long h = hist[u * FB + lane];
    const uint32_t cn = wave_sum<uint32_t>((uint32_t)(h >> 40));
    const unsigned long long mu = wave_sum<unsigned long long>(h & M40);
    if (lane == 0) {
      s_ecnt[u] = cn;
      s_emu[u] = mu;
    }
  }
  __syncthreads();
  // ---- wave 0: the window to list
  if (wave == 0) {
    const uint32_t ec = lane < NEXP ? s_ecnt[lane] : 0u;
    const double em = lane < NEXP ? ldexp((double)s_emu[lane], -lane) : 0.0;
    const uint32_t cc = wave_scan_incl<uint32_t>(ec);
    const double cm = wave_scan_incl<double>(em);
    auto ccof = [&](int u) -> uint32_t { return u < 0 ? 0u : (uint32_t)__shfl((int)cc, u < NEXP ? u : NEXP - 1, 64); };
    auto cmof = [&](int u) -> double { return u < 0 ? 0.0 : __shfl(cm, u < NEXP ? u : NEXP - 1, 64); };
    auto hcnt = [&](int u) -> uint32_t { return (uint32_t)(hist[u * FB + lane] >> 40); };
    auto hmass = [&](int u) -> double { return ldexp((double)(hist[u * FB + lane] & M40), -u); };
    auto cnt_to = [&](int r) -> uint32_t {  // candidates with rel <= r
      if (r < 0) return 0u;
      if (r >= NBIN) r = NBIN - 1;
      const int u = r >> 6;
      return ccof(u - 1) + wave_sum<uint32_t>(lane <= (r & 63) ? hcnt(u) : 0u);
    };
    auto mass_to = [&](int r) -> double {
      if (r < 0) return 0.0;
      if (r >= NBIN) r = NBIN - 1;
      const int u = r >> 6;
      return cmof(u - 1) + wave_sum<double>(lane <= (r & 63) ? hmass(u) : 0.0);
    };
    auto count_cross = [&](uint32_t target) -> int {  // first rel with cnt_to >= target (NBIN: none)
      const int u = first_lane(lane < NEXP && cc >= target);
      if (u >= NEXP) return NBIN;
      const uint32_t cb = wave_scan_incl<uint32_t>(hcnt(u)) + ccof(u - 1);
      const int l = first_lane(cb >= target);
      return u * FB + (l < 64 ? l : 63);
    };
    auto mass_cross = [&](double target) -> int {
      const int u = first_lane(lane < NEXP && cm >= target);
      if (u >= NEXP) return NBIN - 1;
      const double mb = wave_scan_incl<double>(hmass(u)) + cmof(u - 1);
      const int l = first_lane(mb >= target);
      return u * FB + (l < 64 ? l : 63);
    };
    const bool topk = R.top_k > 0, topp = R.top_p < 1.0f, minp = R.min_p > 0.0f;
    int floor_r = NBIN - 1;
    if (minp) {  // the row's min_p cut is at or above this block's: tokens below the block's cut are out
      const float tmax = tval(M, K);
      const float tcut = (float)((double)(tmax / 1024.0f) + R.log2_min_p) * 1024.0f;
      const int rm = btop - (((int)floorf(tcut)) >> 4);
      if (rm < NBIN) floor_r = min(floor_r, max(rm, 0));
    }
    if (topk) {  // the block's share of the row's top K, with room (the resolver verifies the guess)
      const uint32_t kk = R.top_k <= 64 ? (uint32_t)R.top_k : (uint32_t)min(R.top_k, 2 * R.top_k / G + 64);
      floor_r = min(floor_r, count_cross(kk));
    }
    int w0 = 0, w1 = -1, fl = 0;
    if (topk || topp || minp) {
      const uint32_t nfloor = cnt_to(floor_r);
      if (nfloor <= (uint32_t)CAP) {
        w1 = floor_r;  // the whole top set
      } else if (topp) {
        const int rp_ = min(mass_cross((double)R.top_p * mass_to(floor_r)), floor_r);
        const int b = min(floor_r, rp_ + MARGIN);
        if (cnt_to(b) <= (uint32_t)CAP) {
          w1 = b;
        } else {
          int a = max(0, rp_ - MARGIN), bb = b;
          while (a <= bb && cnt_to(bb) - cnt_to(a - 1) > (uint32_t)CAP) {
            if (bb - rp_ >= rp_ - a)
              bb--;
            else
              a++;
          }
          if (a <= bb) {
            w0 = a;
            w1 = bb;
          } else {
            fl |= RF_OVER;
          }
        }
      } else {  // a min_p / top-k floor with more than CAP tokens above it: the bins just above the floor
        int a = max(0, floor_r - 2 * MARGIN);
        while (a <= floor_r && cnt_to(floor_r) - cnt_to(a - 1) > (uint32_t)CAP) a++;
        if (a <= floor_r) {
          w0 = a;
          w1 = floor_r;
        } else {
          fl |= RF_OVER;
        }
      }
    }
    // elements of power of two w0 >> 6 above w0
    uint32_t pc = 0;
    unsigned long long pm = 0;
    if (w0 <= w1 && (w0 & 63)) {
      const int u = w0 >> 6;
      const unsigned long long h = lane < (w0 & 63) ? hist[u * FB + lane] : 0ull;
      pc = wave_sum<uint32_t>((uint32_t)(h >> 40));
      pm = wave_sum<unsigned long long>(h & M40);
    }
    // lowest non-empty bin
    const unsigned long long nzu = __ballot(lane < NEXP && ec > 0);
    const int umin = 63 - __clzll((long long)nzu);
    const unsigned long long nzb = __ballot(hcnt(umin) > 0);
    const int rel_min = umin * FB + (63 - __clzll((long long)nzb));
    const int nwin = w0 <= w1 ? (int)(cnt_to(w1) - cnt_to(w0 - 1)) : 0;
    const uint32_t npos = ccof(NEXP - 1);
    if (lane == 0) {
      s_win[0] = w0;
      s_win[1] = w1;
      s_win[2] = fl | (w0 <= w1 ? RF_WIN : 0);
      s_win[3] = nwin;
      s_win[4] = rel_min;
      s_win[5] = (int)pc;
      s_win[6] = (int)npos;
      s_pm = pm;
    }
  }
  __syncthreads();
  const int w0 = s_win[0], w1 = s_win[1], fl = s_win[2];
  if (fl & RF_WIN) {
    // cursors: exclusive prefix of the bin counts over w0..w1, in rel order
    uint32_t cv[PP];
    uint32_t loc = 0;
#pragma unroll
    for (int k = 0; k < PP; k++) {
      const int r = w0 + tid * PP + k;
      cv[k] = r <= w1 ? (uint32_t)(hist[r] >> 40) : 0u;
      loc += cv[k];
    }
    uint32_t tot;
    const uint32_t incl = block_scan_incl<NWV1, uint32_t>(loc, s_redu, &tot);
    uint32_t run = incl - loc;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PP; k++) {
      const int r = w0 + tid * PP + k;
      if (r <= w1) hist[r] = run;
      run += cv[k];
    }
    __syncthreads();
    uint64_t* EL = (uint64_t*)(rec + HDR_BYTES);
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const uint32_t rel = (rp[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
      if (rel - (uint32_t)w0 <= (uint32_t)(w1 - w0)) {
        const unsigned long long pos = atomicAdd(&hist[rel], 1ull);
        EL[pos] = comp(okey(x[e]), (uint32_t)(lo + BL::local(e)));
      }
    }
  }
  if (tid == 0) {
    H->max_key = okey(M);
    H->max_idx = imax;
    H->c = c;
    H->flags = RF_CAND | RF_SAMP | fl;
    H->rel_max = btop - wm.bin();
    H->rel_min = s_win[4];
    H->w0 = w0;
    H->w1 = w1;
    H->n_pos = (uint32_t)s_win[6];
    H->n_win = (uint32_t)s_win[3];
    H->pcnt = (uint32_t)s_win[5];
    H->pmu = s_pm;
  }
  if (tid < NEXP) {
    H->ecnt[tid] = s_ecnt[tid];
    H->emu[tid] = s_emu[tid];
  }
}

// ---------------------------------------------------------------------------------------------- k_resolve
struct BH {                      // a block's record as the resolver uses it
  uint32_t max_key, max_idx;
  int c, flags, rel_max, rel_min, w0, w1;
  uint32_t n_win, eoff;          // listed elements and their offset in the row's flat element order
  int d;                         // row bin of the block's rel 0: (N - c) * 64
  int mode;                      // kept-mass case of the draw cut: 0 nothing, 1 above-window + listed, 2 all
  int listed;                    // window usable (inside the row window)
};

struct RS {                      // row state (LDS)
  uint32_t max_key, max_idx;
  int N, row_top, Gact, fallback;
  float K, tmax;
  unsigned long long Tlo[MAXG], Thi[MAXG], Alo[MAXG], Ahi[MAXG], Wlo[MAXG], Whi[MAXG], Klo[MAXG], Khi[MAXG];
  uint32_t nT[MAXG], nA[MAXG], nW[MAXG];
  int cR;                        // cut: kept = R < cR, or R == cR and comp >= cC (cR = NR: no cut)
  unsigned long long cC;
  int found;
  unsigned long long t_lo, t_hi; // scratch u128
  int si[8];
};

struct KL {                      // k_resolve LDS views
  unsigned long long *mlo, *mhi; // [NR] row-bin masses (row units), then inclusive prefix
  uint32_t* cnt;                 // [NR] counts, then prefix
  int* good;                     // [NR + 1] good-block difference array, then prefix
  uint64_t* ec;                  // [XN] elements of one bin: comp
  uint32_t* em;                  // [XN] their mantissas
  uint64_t* ep;                  // [XN] inclusive prefix of em
  uint32_t* tab;                 // [BLK] processor table of a rescanned block
  float2* ts;
  BH* bh;
  RS* st;
  u128* red;
  uint32_t* redu;
  uint64_t* red64;
};

__device__ inline u128 ld128(unsigned long long lo, unsigned long long hi) { return ((u128)hi << 64) | lo; }
__device__ inline u128 Cm(const KL& L, int r) { return r < 0 ? (u128)0 : ld128(L.mlo[r], L.mhi[r]); }
__device__ inline uint32_t Cn(const KL& L, int r) { return r < 0 ? 0u : L.cnt[r]; }
__device__ inline bool Good(const KL& L, int r) { return r >= 0 && r < NR && L.good[r] == L.st->Gact; }
// row weight of a mantissa in row bin r: mu * 2^(35 - (r >> 6))
__device__ inline u128 rw(uint32_t mu, int r) { return (u128)mu << (D_EXP - (r >> 6)); }

// Element of the row's flat listed order i -> (block, element)
__device__ inline int block_of(const KL& L, int G, uint32_t i) {
  int a = 0, b = G - 1;
  while (a < b) {
    const int m = (a + b + 1) >> 1;
    if (L.bh[m].eoff <= i)
      a = m;
    else
      b = m - 1;
  }
  return a;
}
struct ElW {
  uint64_t c;
  int r;         // row bin (>= NR: weighs nothing)
  uint32_t mu;
};
__device__ inline ElW el_weigh(uint64_t cmp, const RS& st, const float2* ts) {
  ElW o;
  o.c = cmp;
  const W w = weigh(tval(okey_val(comp_key(cmp)), st.K), ts);
  o.r = st.row_top - w.bin();
  o.mu = w.mu;
  return o;
}

// first row bin whose inclusive prefix reaches target (mass or count): the unique r with C(r) >= t > C(r - 1)
template <bool MASS>
__device__ int first_cross(const KL& L, u128 target) {
  if (threadIdx.x == 0) L.st->found = NR;
  __syncthreads();
  for (int r = threadIdx.x; r < NR; r += NT2) {
    const u128 v = MASS ? Cm(L, r) : (u128)Cn(L, r);
    const u128 p = MASS ? Cm(L, r - 1) : (u128)Cn(L, r - 1);
    if (v >= target && p < target) L.st->found = r;
  }
  __syncthreads();
  const int r = L.st->found;
  __syncthreads();
  return r;
}

// Sorts n (comp, mu) pairs descending by comp (bitonic; n <= XN).  Pads with zeros.
__device__ void sort_bin(const KL& L, int n) {
  int np = 1;
  while (np < n) np <<= 1;
  for (int i = n + threadIdx.x; i < np; i += NT2) {
    L.ec[i] = 0;
    L.em[i] = 0;
  }
  __syncthreads();
  for (int k = 2; k <= np; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < np; i += NT2) {
        const int p = i ^ j;
        if (p > i) {
          const bool desc = (i & k) == 0;
          const uint64_t a = L.ec[i], b = L.ec[p];
          if (desc ? a < b : a > b) {
            L.ec[i] = b;
            L.ec[p] = a;
            const uint32_t t = L.em[i];
            L.em[i] = L.em[p];
            L.em[p] = t;
          }
        }
      }
      __syncthreads();
    }
  }
}

// ---- element sources: the listed windows (fast path) or rescans of the row's logits (fallback)
// Calls fn(cmp, row bin, mu) for every listed element with a nonzero row weight.
template <typename F>
__device__ inline void for_listed(const KL& L, char* ws, int G, int row, F fn) {
  const uint32_t ne = L.bh[G - 1].eoff + L.bh[G - 1].n_win;
  for (uint32_t i = threadIdx.x; i < ne; i += NT2) {
    const int g = block_of(L, G, i);
    const BH& h = L.bh[g];
    if (!h.listed) continue;
    const uint64_t cmp = ((const uint64_t*)(rec_of(ws, G, row, g) + HDR_BYTES))[i - h.eoff];
    const ElW w = el_weigh(cmp, *L.st, L.ts);
    if (w.r < NR) fn(g, cmp, w.r, w.mu);
  }
}
// Calls fn(block, cmp, row bin, mu) for every candidate of the row with a nonzero row weight, block by block.
template <int DT, typename F>
__device__ inline void for_rescan(const KL& L, const qws_batch& B, const qws_row& R, int row, int G, F fn) {
  using BL = Blk<DT, NT2>;
  for (int g = 0; g < G; g++) {
    if (L.bh[g].d >= NR || !(L.bh[g].flags & RF_CAND)) continue;  // nothing of this block weighs in the row
    const int lo = g * BLK, hi = min(B.V, lo + BLK);
    float x[BL::EPT];
    load_processed<DT, NT2>(B, R, row, lo, hi, L.tab, x);
#pragma unroll
    for (int e = 0; e < BL::EPT; e++) {
      if (x[e] == -INFINITY) continue;
      const W w = weigh(tval(x[e], L.st->K), L.ts);
      const int r = L.st->row_top - w.bin();
      if (r < NR) fn(g, comp(okey(x[e]), (uint32_t)(lo + BL::local(e))), r, w.mu);
    }
    __syncthreads();
  }
}

// Gathers the elements of row bin r with comp >= cmin into L.ec / L.em, sorted descending.  Returns the count,
// or -1 when the bin holds more than XN of them.
template <int DT>
__device__ int gather_bin(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int G, int r, uint64_t cmin, bool rescan) {
  if (threadIdx.x == 0) L.st->si[0] = 0;
  __syncthreads();
  auto put = [&](int, uint64_t cmp, int rr, uint32_t mu) {
    if (rr != r || cmp < cmin) return;
    const int p = atomicAdd(&L.st->si[0], 1);
    if (p < XN) {
      L.ec[p] = cmp;
      L.em[p] = mu;
    }
  };
  if (rescan)
    for_rescan<DT>(L, B, R, row, G, put);
  else
    for_listed(L, ws, G, row, put);
  __syncthreads();
  const int n = L.st->si[0];
  __syncthreads();
  if (n > XN) return -1;
  sort_bin(L, n);
  // inclusive prefix of the mantissas in sorted order (two elements per thread; XN = 2 * NT2)
  const int i0 = threadIdx.x * 2;
  const uint64_t a = i0 < n ? L.em[i0] : 0ull, b = i0 + 1 < n ? L.em[i0 + 1] : 0ull;
  uint64_t tot;
  const uint64_t inc = block_scan_incl<NWV2, uint64_t>(a + b, L.red64, &tot);
  if (i0 < n) L.ep[i0] = inc - b;
  if (i0 + 1 < n) L.ep[i0 + 1] = inc;
  __syncthreads();
  return n;
}
static_assert(XN == 2 * NT2, "two bin elements per resolver thread");

// Builds the row-bin arrays: masses, counts and the good-block difference array.  Fast path: from the records
// (exact at good bins).  Fallback: from rescans (exact everywhere).
template <int DT>
__device__ void build_bins(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int G, bool rescan) {
  RS& st = *L.st;
  for (int r = threadIdx.x; r < NR; r += NT2) {
    L.mlo[r] = 0;
    L.mhi[r] = 0;
    L.cnt[r] = 0;
    L.good[r] = 0;
  }
  if (threadIdx.x == 0) L.good[NR] = 0;
  for (int g = threadIdx.x; g < G; g += NT2) {
    st.Wlo[g] = 0;
    st.Whi[g] = 0;
    st.nW[g] = 0;
  }
  __syncthreads();
  if (rescan) {
    for_rescan<DT>(L, B, R, row, G, [&](int, uint64_t, int r, uint32_t mu) {
      atomic_add_u128(&L.mlo[r], &L.mhi[r], rw(mu, r));
      atomicAdd(&L.cnt[r], 1u);
    });
    if (threadIdx.x == 0) L.good[0] = st.Gact;  // every bin is exact
    __syncthreads();
    return;
  }
  for_listed(L, ws, G, row, [&](int g, uint64_t, int r, uint32_t mu) {
    const u128 w = rw(mu, r);
    atomic_add_u128(&L.mlo[r], &L.mhi[r], w);
    atomicAdd(&L.cnt[r], 1u);
    atomic_add_u128(&st.Wlo[g], &st.Whi[g], w);
    atomicAdd(&st.nW[g], 1u);
  });
  __syncthreads();
  // per block: good intervals and the lumps for the mass above its window and below it
  for (int g = threadIdx.x; g < G; g += NT2) {
    const BH& h = L.bh[g];
    auto good_iv = [&](int a, int b) {
      a = max(a, 0);
      b = min(b, NR - 1);
      if (a > b) return;
      atomicAdd(&L.good[a], 1);
      atomicSub(&L.good[b + 1], 1);
    };
    if (!(h.flags & RF_CAND) || h.d + h.rel_max >= NR) {  // nothing of this block weighs in the row
      good_iv(0, NR - 1);
      continue;
    }
    good_iv(0, h.d + h.rel_max - 1);
    if (h.listed) good_iv(h.d + h.w0, h.d + h.w1);
    good_iv(h.d + h.rel_min + 1, NR - 1);
    const u128 T = ld128(st.Tlo[g], st.Thi[g]), A = ld128(st.Alo[g], st.Ahi[g]), Wm = ld128(st.Wlo[g], st.Whi[g]);
    if (h.listed && h.w0 > 0 && (A != 0 || st.nA[g])) {
      const int r = h.d + h.w0 - 1;
      atomic_add_u128(&L.mlo[r], &L.mhi[r], A);
      atomicAdd(&L.cnt[r], st.nA[g]);
    }
    const u128 Bm = h.listed ? T - A - Wm : T;
    const uint32_t nB = h.listed ? st.nT[g] - st.nA[g] - st.nW[g] : st.nT[g];
    if (Bm != 0 || nB) {
      const int r = min(h.d + h.rel_min, NR - 1);
      atomic_add_u128(&L.mlo[r], &L.mhi[r], Bm);
      atomicAdd(&L.cnt[r], nB);
    }
  }
  __syncthreads();
}

// Inclusive prefixes over the row bins (mass, count, good).
__device__ void scan_bins(const KL& L) {
  constexpr int PR = (NR + NT2 - 1) / NT2;
  const int r0 = threadIdx.x * PR;
  u128 m[PR];
  uint32_t n[PR];
  int gd[PR];
  u128 ms = 0;
  uint32_t ns = 0;
  int gs = 0;
#pragma unroll
  for (int k = 0; k < PR; k++) {
    const int r = r0 + k;
    m[k] = r < NR ? ld128(L.mlo[r], L.mhi[r]) : (u128)0;
    n[k] = r < NR ? L.cnt[r] : 0u;
    gd[k] = r < NR ? L.good[r] : 0;
    ms += m[k];
    ns += n[k];
    gs += gd[k];
  }
  u128 mt;
  const u128 mi = block_scan_incl_u128<NWV2>(ms, L.red, &mt);
  uint32_t nt;
  const uint32_t ni = block_scan_incl<NWV2, uint32_t>(ns, L.redu, &nt);
  int gt;
  const int gi = (int)block_scan_incl<NWV2, uint32_t>((uint32_t)gs, L.redu, (uint32_t*)&gt);
  u128 mr = mi - ms;
  uint32_t nr = ni - ns;
  int gr = gi - gs;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < PR; k++) {
    const int r = r0 + k;
    mr += m[k];
    nr += n[k];
    gr += gd[k];
    if (r < NR) {
      L.mlo[r] = (unsigned long long)mr;
      L.mhi[r] = (unsigned long long)(mr >> 64);
      L.cnt[r] = nr;
      L.good[r] = gr;
    }
  }
  __syncthreads();
}

// Rescans block g and returns the token whose kept-mass interval (index order) holds the local target tl, or -1.
template <int DT>
__device__ int draw_in_block(const KL& L, const qws_batch& B, const qws_row& R, int row, int g, u128 tl) {
  using BL = Blk<DT, NT2>;
  const RS& st = *L.st;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  float x[BL::EPT];
  load_processed<DT, NT2>(B, R, row, lo, hi, L.tab, x);
  if (threadIdx.x == 0) L.st->si[7] = -1;
  __syncthreads();
  u128 run = 0;
#pragma unroll
  for (int s = 0; s < BL::S; s++) {
    u128 w[BL::VEC];
    u128 loc = 0;
#pragma unroll
    for (int j = 0; j < BL::VEC; j++) {
      const int e = s * BL::VEC + j;
      w[j] = 0;
      if (x[e] != -INFINITY) {
        const W ww = weigh(tval(x[e], st.K), L.ts);
        const int r = st.row_top - ww.bin();
        if (r < NR && (r < st.cR || (r == st.cR && comp(okey(x[e]), (uint32_t)(lo + BL::local(e))) >= st.cC))) w[j] = rw(ww.mu, r);
      }
      loc += w[j];
    }
    u128 tot;
    const u128 inc = block_scan_incl_u128<NWV2>(loc, L.red, &tot);
    u128 c0 = run + inc - loc;
#pragma unroll
    for (int j = 0; j < BL::VEC; j++) {
      const u128 c1 = c0 + w[j];
      if (w[j] && c0 <= tl && tl < c1) L.st->si[7] = lo + BL::local(s * BL::VEC + j);
      c0 = c1;
    }
    run += tot;
  }
  __syncthreads();
  const int tok = L.st->si[7];
  __syncthreads();
  return tok;
}

// Dense probabilities of the kept set (test-hook path), by rescans.
template <int DT>
__device__ void write_probs(const KL& L, const qws_batch& B, const qws_row& R, int row, int G, u128 S2) {
  const RS& st = *L.st;
  const double S2d = (double)(uint64_t)(S2 >> 64) * 18446744073709551616.0 + (double)(uint64_t)S2;
  for_rescan<DT>(L, B, R, row, G, [&](int, uint64_t cmp, int r, uint32_t mu) {
    if (r < st.cR || (r == st.cR && cmp >= st.cC)) {
      const u128 w = rw(mu, r);
      B.out_probs[(size_t)row * B.V + comp_idx(cmp)] = (float)(((double)(uint64_t)(w >> 64) * 18446744073709551616.0 + (double)(uint64_t)w) / S2d);
    }
  });
}

// The row from the prepared bins.  Returns false when a boundary is not pinned (fast path only).
template <int DT>
__device__ bool resolve_row(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int G, bool rescan) {
  RS& st = *L.st;
  const int tid = threadIdx.x;
  const u128 Stot = Cm(L, NR - 1);
  const uint32_t Npos = Cn(L, NR - 1);
  int cR = NR;
  uint64_t cC = 0;
  u128 S = Stot;
  uint32_t Nk = Npos;
  // ---- min_p: keep t >= t_cut
  if (R.min_p > 0.0f) {
    const float tcut = (float)((double)(st.tmax / 1024.0f) + R.log2_min_p) * 1024.0f;
    const int rm = st.row_top - (((int)floorf(tcut)) >> 4);
    if (rm < NR) {
      if (!rescan && !Good(L, max(rm, 0))) return false;
      const int n = gather_bin<DT>(L, B, R, ws, row, G, max(rm, 0), 0, rescan);
      if (n < 0) return false;  // (the rescan path never overflows a bin of a min_p cut: see DESIGN)
      // kept in the bin: t >= tcut, a prefix of the sorted elements
      if (tid == 0) st.si[1] = 0;
      __syncthreads();
      for (int i = tid; i < n; i += NT2) {
        const bool in = tval(okey_val(comp_key(L.ec[i])), st.K) >= tcut;
        const bool nx = i + 1 < n && tval(okey_val(comp_key(L.ec[i + 1])), st.K) >= tcut;
        if (in && !nx) st.si[1] = i + 1;
      }
      __syncthreads();
      const int k = st.si[1];
      cR = max(rm, 0);
      cC = k ? L.ec[k - 1] : ~0ull;
      S = Cm(L, cR - 1) + (k ? ((u128)L.ep[k - 1] << (D_EXP - (cR >> 6))) : (u128)0);
      Nk = Cn(L, cR - 1) + (uint32_t)k;
      __syncthreads();
    }
  }
  // ---- top-k over the min_p survivors
  if (R.top_k > 0 && Nk > (uint32_t)R.top_k) {
    const int rk = first_cross<false>(L, (u128)(uint32_t)R.top_k);
    if (!rescan && !Good(L, rk)) return false;
    const int n = gather_bin<DT>(L, B, R, ws, row, G, rk, rk == cR ? cC : 0, rescan);
    if (n < 0) return false;
    const int m = R.top_k - (int)Cn(L, rk - 1);  // 1-based position inside the bin
    cR = rk;
    cC = L.ec[m - 1];
    S = Cm(L, rk - 1) + ((u128)L.ep[m - 1] << (D_EXP - (rk >> 6)));
    __syncthreads();
  }
  // ---- top-p over the kept set: the first rank position whose inclusive mass reaches thr
  u128 S2 = S;
  if (R.top_p < 1.0f) {
    const uint64_t TP = (uint64_t)floor((double)R.top_p * 4294967296.0);
    u128 thr = mul_shr_ceil(S, TP, 32);
    if (thr == 0) thr = 1;
    const int rp = first_cross<true>(L, thr);
    if (!rescan && !Good(L, rp)) return false;
    const int n = gather_bin<DT>(L, B, R, ws, row, G, rp, rp == cR ? cC : 0, rescan);
    if (n < 0) return false;
    // the first sorted element whose inclusive mass reaches thr (the last one when rounding leaves none)
    const u128 base = Cm(L, rp - 1);
    const int sh = D_EXP - (rp >> 6);
    if (tid == 0) st.si[1] = n - 1;
    __syncthreads();
    for (int i = tid; i < n; i += NT2) {
      const bool reach = base + ((u128)L.ep[i] << sh) >= thr;
      const bool before = i > 0 && base + ((u128)L.ep[i - 1] << sh) >= thr;
      if (reach && !before) st.si[1] = i;
    }
    __syncthreads();
    const int k = st.si[1];
    cR = rp;
    cC = L.ec[k];
    S2 = base + ((u128)L.ep[k] << sh);
    __syncthreads();
  }
  if (tid == 0) {
    st.cR = cR;
    st.cC = cC;
  }
  __syncthreads();
  // ---- kept mass per block (index order) and the block of the draw
  const uint32_t u24 = draw_u24(R.seed, R.position, R.stream, R.row_key, 0);
  const u128 tt = mul_shr_floor(S2, u24, 24);
  for (int g = tid; g < G; g += NT2) {
    st.Klo[g] = 0;
    st.Khi[g] = 0;
  }
  __syncthreads();
  if (rescan) {
    for_rescan<DT>(L, B, R, row, G, [&](int g, uint64_t cmp, int r, uint32_t mu) {
      if (r < cR || (r == cR && cmp >= cC)) atomic_add_u128(&st.Klo[g], &st.Khi[g], rw(mu, r));
    });
  } else {
    for (int g = tid; g < G; g += NT2) {
      BH& h = L.bh[g];
      int mode = 0;
      if ((h.flags & RF_CAND) && h.d + h.rel_max < NR) {
        if (cR >= NR || cR > h.d + h.rel_min) mode = 2;
        else if (cR < h.d + h.rel_max) mode = 0;
        else mode = 1;  // cR inside the listed window (cR is good)
      }
      h.mode = mode;
      if (mode == 2) {
        st.Klo[g] = st.Tlo[g];
        st.Khi[g] = st.Thi[g];
      } else if (mode == 1) {
        st.Klo[g] = st.Alo[g];
        st.Khi[g] = st.Ahi[g];
      }
    }
    __syncthreads();
    for_listed(L, ws, G, row, [&](int g, uint64_t cmp, int r, uint32_t mu) {
      if (L.bh[g].mode == 1 && (r < cR || (r == cR && cmp >= cC))) atomic_add_u128(&st.Klo[g], &st.Khi[g], rw(mu, r));
    });
  }
  __syncthreads();
  if (tid == 0) {
    u128 run = 0;
    int gs = -1;
    for (int g = 0; g < G; g++) {
      const u128 k = ld128(st.Klo[g], st.Khi[g]);
      if (gs < 0 && k != 0 && tt < run + k) {
        gs = g;
        const u128 tl = tt - run;
        st.t_lo = (unsigned long long)tl;
        st.t_hi = (unsigned long long)(tl >> 64);
      }
      run += k;
    }
    st.si[2] = gs;
  }
  __syncthreads();
  const int gs = st.si[2];
  const u128 tl = ld128(st.t_lo, st.t_hi);
  __syncthreads();
  int tok = -1;
  if (gs >= 0) tok = draw_in_block<DT>(L, B, R, row, gs, tl);
  if (B.out_probs) write_probs<DT>(L, B, R, row, G, S2);
  if (tid == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = rescan ? 1 : 0;
  }
  return true;
}

template <int DT>
__global__ void __launch_bounds__(NT2) k_resolve(qws_batch B, int G, char* ws) {
  __shared__ unsigned long long s_mlo[NR], s_mhi[NR];
  __shared__ uint32_t s_cnt[NR];
  __shared__ int s_good[NR + 1];
  __shared__ uint64_t s_ec[XN];
  __shared__ uint32_t s_em[XN];
  __shared__ uint64_t s_ep[XN];
  __shared__ __attribute__((aligned(16))) uint32_t s_tab[BLK];
  __shared__ __attribute__((aligned(16))) float2 s_ts[1024];
  __shared__ BH s_bh[MAXG];
  __shared__ RS s_st;
  __shared__ u128 s_red[NWV2];
  __shared__ uint32_t s_redu[NWV2];
  __shared__ uint64_t s_red64[NWV2];
  KL L;
  L.mlo = s_mlo;
  L.mhi = s_mhi;
  L.cnt = s_cnt;
  L.good = s_good;
  L.ec = s_ec;
  L.em = s_em;
  L.ep = s_ep;
  L.tab = s_tab;
  L.ts = s_ts;
  L.bh = s_bh;
  L.st = &s_st;
  L.red = s_red;
  L.redu = s_redu;
  L.red64 = s_red64;
  RS& st = s_st;
  const int row = blockIdx.x, tid = threadIdx.x;
  const qws_row R = B.rows[row];
  if (tid < 512) ((uint4*)s_ts)[tid] = ((const uint4*)EXP2_TS)[tid];
  // ---- block headers, the row's best
  uint64_t best = 0;
  for (int g = tid; g < G; g += NT2) {
    const Rec* H = (const Rec*)rec_of(ws, G, row, g);
    BH h;
    h.max_key = H->max_key;
    h.max_idx = H->max_idx;
    h.flags = H->flags;
    h.c = H->c;
    h.rel_max = H->rel_max;
    h.rel_min = H->rel_min;
    h.w0 = H->w0;
    h.w1 = H->w1;
    h.n_win = (h.flags & RF_WIN) ? H->n_win : 0u;
    h.d = 0;
    h.mode = 0;
    h.listed = 0;
    s_bh[g] = h;
    if (h.flags & RF_CAND) {
      const uint64_t cv = comp(h.max_key, h.max_idx);
      best = cv > best ? cv : best;
    }
  }
  best = block_max_u64<NWV2>(best, s_red64);
  const float K = kscale(R.temperature);
  if (best == 0 || !(R.temperature > 0.0f) || !(K < INFINITY)) {  // no candidate, or a greedy row
    if (tid == 0) {
      B.out_tokens[row] = best == 0 ? 0 : (int)comp_idx(best);
      if (B.out_info) B.out_info[row] = 2;
    }
    return;
  }
  if (tid == 0) {
    st.max_key = comp_key(best);
    st.max_idx = comp_idx(best);
    st.K = K;
    st.tmax = tval(okey_val(st.max_key), K);
    const W w = weigh(st.tmax, ts_const());
    st.N = w.n();
    st.row_top = st.N * FB + (FB - 1);
    st.fallback = 0;
  }
  __syncthreads();
  // ---- per block: realigned totals, the mass above the window, the listed-element offsets
  for (int g = tid; g < G; g += NT2) {
    BH& h = s_bh[g];
    u128 T = 0, A = 0;
    uint32_t nT = 0, nA = 0;
    int active = 0;
    if (h.flags & RF_CAND) {
      h.d = (st.N - h.c) * FB;
      active = h.d + h.rel_max < NR;
      const Rec* H = (const Rec*)rec_of(ws, G, row, g);
      const int dn = st.N - h.c;
      for (int e = 0; e < NEXP; e++) {
        const int sh = D_EXP - dn - e;
        if (sh < 0) break;
        const u128 m = (u128)H->emu[e] << sh;
        T += m;
        nT += H->ecnt[e];
        if ((h.flags & RF_WIN) && e < (h.w0 >> 6)) {
          A += m;
          nA += H->ecnt[e];
        }
      }
      if ((h.flags & RF_WIN) && (h.w0 & 63)) {
        const int sh = D_EXP - dn - (h.w0 >> 6);
        if (sh >= 0) {
          A += (u128)H->pmu << sh;
          nA += H->pcnt;
        }
      }
      // a usable window lies inside the row window; clip it to the block's occupied bins
      if ((h.flags & RF_WIN) && active && h.d + h.w0 < NR) {
        h.listed = 1;
        if (h.w0 < h.rel_max) {
          h.w0 = h.rel_max;
          A = 0;
          nA = 0;
        }
        if (h.w1 > h.rel_min) h.w1 = h.rel_min;
      }
    }
    st.Tlo[g] = (unsigned long long)T;
    st.Thi[g] = (unsigned long long)(T >> 64);
    st.Alo[g] = (unsigned long long)A;
    st.Ahi[g] = (unsigned long long)(A >> 64);
    st.nT[g] = nT;
    st.nA[g] = nA;
    if (!active) h.listed = 0;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t off = 0;
    int ga = 0;
    for (int g = 0; g < G; g++) {
      s_bh[g].eoff = off;
      off += s_bh[g].n_win;
      ga++;
    }
    st.Gact = ga;  // every block counts once in the good-block difference array
  }
  __syncthreads();
  build_bins<DT>(L, B, R, ws, row, G, false);
  scan_bins(L);
  if (resolve_row<DT>(L, B, R, ws, row, G, false)) return;
  __syncthreads();
  build_bins<DT>(L, B, R, ws, row, G, true);
  scan_bins(L);
  if (!resolve_row<DT>(L, B, R, ws, row, G, true) && tid == 0) {  // a boundary bin beyond XN elements
    B.out_tokens[row] = -1;
    if (B.out_info) B.out_info[row] = -1;
  }
}

}  // namespace qws

// ---------------------------------------------------------------------------------------------- launcher
namespace qws {
// Optional launch timing (profiling only): events recorded around each kernel of qws_sample.
struct Timing {
  bool on = false;
  int n = 0;
  static constexpr int CAPN = 4096;
  hipEvent_t ev[CAPN][3];
  bool made = false;
};
static Timing g_timing;

static int blocks_of(int V) { return (V + BLK - 1) / BLK; }

template <int DT>
static hipError_t launch(const qws_batch& b, int G, char* ws, hipStream_t st) {
  const bool tm = g_timing.on && g_timing.n < Timing::CAPN;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][0], st);
  hipLaunchKernelGGL((k_scan<DT>), dim3(b.B * G), dim3(NT1), 0, st, b, G, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][1], st);
  hipLaunchKernelGGL((k_resolve<DT>), dim3(b.B), dim3(NT2), 0, st, b, G, ws);
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
  return (size_t)B * qws::blocks_of(V) * qws::REC_BYTES;
}

extern "C" int qws_sample(const qws_batch* b, void* ws, size_t ws_bytes, void* stream) {
  using namespace qws;
  if (!b || !b->logits || !b->rows || !b->out_tokens || !ws) return QWS_ERR_INVALID;
  if (b->B < 1 || b->V < 8 || (b->V & 7) || (b->row_stride & 7) || b->row_stride < 0) return QWS_ERR_INVALID;
  if (b->row_stride != 0 && b->row_stride < b->V) return QWS_ERR_INVALID;
  if (b->dtype != QWS_DTYPE_F32 && b->dtype != QWS_DTYPE_BF16) return QWS_ERR_INVALID;
  if (((uintptr_t)b->logits & 15) || ((uintptr_t)ws & 255)) return QWS_ERR_INVALID;
  if (b->masks && b->mask_words * 32LL < b->V) return QWS_ERR_INVALID;
  const int G = blocks_of(b->V);
  if (G > MAXG) return QWS_ERR_NOT_SUPPORTED;
  if (ws_bytes < (size_t)b->B * G * REC_BYTES) return QWS_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  char* w = (char*)ws;
  const hipError_t e = b->dtype == QWS_DTYPE_F32 ? launch<QWS_DTYPE_F32>(*b, G, w, st) : launch<QWS_DTYPE_BF16>(*b, G, w, st);
  return (int)e;
}
