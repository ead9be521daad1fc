// The record format of the sampling kernels and k_resolve, shared by qws_sample.hip (k_scan, the sampling rows'
// k_resolve) and qws_verify.hip (the verify rows' k_resolve, instantiated there so that each kernel family keeps its
// own code object).  The overview of both kernels is at the top of qws_sample.hip.
#pragma once
#include <math.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "qws_rows.h"

namespace qws {

constexpr int NT1S = 512, NT1L = 1024;        // k_scan workgroups: 3 per CU; one per CU when the grid fits one round
constexpr int NXCD = 8;                      // accelerator complex dies (XCDs), each with its own L2
// (row, block) items of k_scan per XCD: an equal share of the grid; with fewer rows than XCDs, a whole row (G items,
// one workgroup per CU of the XCD), so that each row's blocks and its k_resolve workgroup share one L2
__host__ __device__ inline int scan_chunk(int B, int G) { return B < NXCD && G <= 32 ? G : (B * G + NXCD - 1) / NXCD; }
inline unsigned scan_grid(int B, int G) { return (unsigned)(NXCD * scan_chunk(B, G)); }
constexpr int NT2 = 512, NWV2 = NT2 / 64;    // k_resolve workgroup
// k_resolve's grid: workgroup i takes row (i mod 8) * ceil(B / 8) + i / 8, the row k_scan ran on workgroup i's XCD
inline unsigned resolve_grid(int B) { return (unsigned)(NXCD * ((B + NXCD - 1) / NXCD)); }
constexpr int CAP = 1024;                    // elements a block may list
// top-p: fine bins listed at most on either side of the block's own boundary (as many as the list holds): a flat
// block's boundary is close to the row's, a peaked block's (its top CTOP elements carry a real share of its mass) far
// less so: its window widens to MARGIN_NEAR, then, when that fits whole, to MARGIN, trimmed to the list's capacity from
// below first (a row's cut tends to lie above a peaked block's own boundary, and bins above it hold fewer elements)
constexpr int MARGIN_FLAT = 6, MARGIN_NEAR = 31, MARGIN = 100;
constexpr int CTOP = 256;                    // elements of a block's top bins listed beside a window further down
constexpr int MAXG = 64;                     // blocks per row (V <= 524,288)
constexpr int NR = NBIN;                     // row bins with a nonzero weight (row-relative, 0 = the top)
constexpr int XN = 4096;                     // elements of one bin k_resolve holds in LDS
constexpr unsigned long long M40 = (1ull << 40) - 1;

// ---------------------------------------------------------------------------------------------- block record
enum : int { RF_CAND = 1, RF_SAMP = 2 };
// Bins of a block are top-down: rel = (c * 64 + 63) - fine bin, so rel 0..63 is the power of two 2^c of the block's
// best and rel >> 6 = e counts powers of two below it.  Elements with rel >= NBIN weigh nothing in any row.
struct Rec {
  uint32_t max_key, max_idx;     // best candidate (okey, lowest index); KEY_NEGINF: none
  int c, flags;                  // power of two of the best; RF_*
  int nbw;                       // bins written: rel 0 .. nbw - 1 (every bin a cut of any row can fall in)
  int w0, w1, wa, ea;            // listed bins: rel in [w0, w1] with rel <= wa or rel >= ea (none when w0 > w1)
  int n_list, n_patch, pad0;     // listed elements; processed touched tokens recorded (-1: more than TCAP)
  uint32_t pad1[4];
  uint32_t ecnt[NEXP];           // candidates of power of two e = rel >> 6
  unsigned long long emu[NEXP];  // their summed mantissas (< 2^37)
};
constexpr size_t HDR_BYTES = 512;
static_assert(sizeof(Rec) <= HDR_BYTES && offsetof(Rec, ecnt) == 64 && offsetof(Rec, emu) % 8 == 0, "record header");
// then the bin words: mantissa sum (bits 0..36) | count (37..50) | list offset (51..61) | listed (62), then the
// listed elements comp(key, index), bucketed by bin, then the patches {local index, processed value}
constexpr size_t BIN_OFF = HDR_BYTES;
constexpr size_t EL_OFF = BIN_OFF + (size_t)NBIN * 8;
constexpr size_t PATCH_OFF = EL_OFF + (size_t)CAP * 8;
constexpr size_t REC_BYTES = PATCH_OFF + (size_t)TCAP * 8;
static_assert(CAP <= 2048 && BLK < (1 << 14), "bin word fields");
__device__ inline char* rec_of(char* ws, int G, int row, int g) { return ws + ((size_t)row * G + g) * REC_BYTES; }
constexpr unsigned long long BW_MU = (1ull << 37) - 1;
__device__ inline uint32_t bw_cnt(unsigned long long w) { return (uint32_t)(w >> 37) & 0x3FFFu; }
__device__ inline unsigned long long bw_mu(unsigned long long w) { return w & BW_MU; }
__device__ inline uint32_t bw_off(unsigned long long w) { return (uint32_t)(w >> 51) & 0x7FFu; }
__device__ inline bool bw_listed(unsigned long long w) { return (w >> 62) & 1ull; }

// ---------------------------------------------------------------------------------------------- block searches
// Wave-level searches over a block's LDS histogram (hist[rel] = count << 40 | mantissa sum) and its per-power sums,
// by all 64 lanes of one wave: first the power of two, then the fine bin inside it.
// Inclusive cumulative count up to bin r (0 for r < 0)
__device__ inline uint32_t blk_cnt_to(const unsigned long long* hist, const uint32_t* ecnt, int r) {
  if (r < 0) return 0u;
  r = min(r, NBIN - 1);
  const int lane = lane_id(), p = r >> 6;
  uint32_t v = lane < p ? ecnt[lane] : 0u;
  v += lane <= (r & 63) ? (uint32_t)(hist[p * FB + lane] >> 40) : 0u;
  return wave_sum<uint32_t>(v);
}
// approximate mass (relative to the block's top power of two) up to bin r
__device__ inline float blk_mass_to(const unsigned long long* hist, const unsigned long long* emu, int r) {
  if (r < 0) return 0.0f;
  r = min(r, NBIN - 1);
  const int lane = lane_id(), p = r >> 6;
  float v = lane < p ? ldexpf((float)emu[lane], -lane) : 0.0f;
  v += lane <= (r & 63) ? ldexpf((float)(hist[p * FB + lane] & M40), -p) : 0.0f;
  return wave_sum<float>(v);
}
// first bin whose inclusive cumulative count reaches tgt (NBIN when none)
__device__ inline int blk_cross_cnt(const unsigned long long* hist, const uint32_t* ecnt, uint32_t tgt) {
  const int lane = lane_id();
  const uint32_t pc = lane < NEXP ? ecnt[lane] : 0u;
  const uint32_t inc = wave_scan_incl<uint32_t>(pc);
  const int p = first_lane(lane < NEXP && inc >= tgt);
  if (p >= NEXP) return NBIN;
  const uint32_t base = readlane<uint32_t>(inc - pc, p);
  const uint32_t fi = wave_scan_incl<uint32_t>((uint32_t)(hist[p * FB + lane] >> 40)) + base;
  const int f = first_lane(fi >= tgt);
  return p * FB + min(f, 63);
}
// first bin whose inclusive cumulative approximate mass reaches tgt (NBIN when none)
__device__ inline int blk_cross_mass(const unsigned long long* hist, const unsigned long long* emu, float tgt) {
  const int lane = lane_id();
  const float pm = lane < NEXP ? ldexpf((float)emu[lane], -lane) : 0.0f;
  const float inc = wave_scan_incl<float>(pm);
  const int p = first_lane(lane < NEXP && inc >= tgt);
  if (p >= NEXP) return NBIN;
  const float base = readlane<float>(inc - pm, p);
  const float fi = wave_scan_incl<float>(ldexpf((float)(hist[p * FB + lane] & M40), -p)) + base;
  const int f = first_lane(fi >= tgt);
  return p * FB + min(f, 63);
}

// ---------------------------------------------------------------------------------------------- k_resolve
// One workgroup per row.  Global loads come in few parallel rounds (the headers; the fine bins of one power of two of
// every block; one bin's listed elements; the block of the draw); everything else runs from LDS.
constexpr int NBK = 256;         // buckets of a round of the in-bin selection
constexpr int XG = 3072;         // elements of one bin held in LDS (a larger bin is streamed from its sources)
static_assert(MAXG * HDR_BYTES <= (size_t)MAXG * FB * 8, "the headers are staged in the fine-bin region");
static_assert(BLK / NT2 == 16, "a thread's 16 staged tokens start at word 17 t");

struct BI {                      // a block as the resolver uses it
  uint32_t max_key, max_idx;
  int c, flags, nbw, n_patch;
  int dn;                        // N - c (row powers of two above the block's top one); -1: nothing of it weighs in the row
  int gcnt, goff, gsrc, gofs;    // the bin being gathered: the block's count, list offset, source (0 none, 1 list, 2 rescan),
                                 // first slot in the gathered list
  int w0, w1, wa, ea;            // the block's listed bins (its record header's window)
  int n_list, wcnt;              // its listed elements; its candidates inside the row's weight window
};

struct RS {                      // row state (LDS)
  int G, N, row_top;
  int fpow;                      // row power of two whose fine bins are staged (-1: none)
  int gbin, gn, gl, gstaged;     // the gathered bin: row bin, elements, listed ones, held in LDS
  int gres;                      // blocks of the gathered bin rescanned (their window missed it)
  unsigned long long gfast;      // bit g: block g is rescanned straight from its raw logits (no mask, no processed tokens)
  unsigned long long gslow;      // bit g: block g is rescanned through the staged block (mask or processed tokens)
  int rescans;                   // blocks rescanned because their window missed a bin
  float K;
  unsigned long long best;
  uint32_t Rc[NEXP];             // the row's candidates per power of two (row power e: 2^(N - e))
  unsigned long long Rm[NEXP];   // their summed mantissas (< 2^42)
  uint32_t fcnt[FB];             // the staged power's fine bins over the row: counts, mantissa sums
  unsigned long long fmu[FB];
  uint32_t pcnt[NWV2][FB];       // stage_power's per-wave partial sums
  unsigned long long pmu[NWV2][FB];
  int si[8];
  unsigned long long su[8];
  unsigned long long kmin, kmax;
  unsigned long long gmin, gmax;  // comp range of the gathered bin (held in LDS)
  unsigned long long wmn[NWV2], wmx[NWV2];  // per-wave comp ranges of a bin gathered by select_listed
  uint32_t bcnt[NBK];
  unsigned long long bsum[NBK];
  unsigned long long Klo[MAXG], Khi[MAXG];  // kept mass per block (row units)
  uint64_t xs[64], xv[64];
  uint32_t fbc[NBK];             // topp_cut_fast's buckets (zeroed at the start of k_resolve, used once per row)
  unsigned long long fbs[NBK];
  int fxn;                       // its crossing bucket's elements
  uint64_t fxs[64], fxv[64];
};

struct RL {                      // k_resolve LDS views
  BI* bi;
  RS* st;
  float2* ts;
  uint32_t* big;                 // [BLK]: a staged block
  unsigned long long* fb;        // [MAXG][FB]: the staged power's bin words per block (first: the staged headers)
  unsigned long long* emu;       // [MAXG][NEXP]: the blocks' per-power mantissa sums
  uint64_t* ec;                  // [XG] gathered elements: comp
  uint32_t* em;                  //                          mantissa
  int* nt;
  u128* red;
};

__device__ inline u128 ld128(unsigned long long lo, unsigned long long hi) { return ((u128)hi << 64) | lo; }
// row weight of one mantissa in row bin r (< 2^59)
__device__ inline uint64_t rw1(uint32_t mu, int r) { return (uint64_t)mu << (D_EXP - (r >> 6)); }
__device__ inline const QWS_G uint64_t* els_of(char* ws, int G, int row, int g) { return gmem((const uint64_t*)(rec_of(ws, G, row, g) + EL_OFF)); }
__device__ inline const QWS_G unsigned long long* bins_of(char* ws, int G, int row, int g) {
  return gmem((const unsigned long long*)(rec_of(ws, G, row, g) + BIN_OFF));
}
// The smallest sh with (range >> sh) < NBK: the bucket width of a selection round over a comp range
__device__ inline int bucket_shift(uint64_t range) {
  const int bits = range ? 64 - __clzll((long long)range) : 0;
  return max(bits - 8, 0);
}

// Sum / min / max of one value per thread over the workgroup, via one atomic per wave (st.su[7] / kmin / kmax); the
// caller reads the result after the barrier these end with.
__device__ inline void block_add_u64(RS& st, unsigned long long v) {
  if (threadIdx.x == 0) st.su[7] = 0ull;
  bar();
  v = wave_sum<unsigned long long>(v);
  if (lane_id() == 0 && v) atomicAdd(&st.su[7], v);
  bar();
}
__device__ inline void block_range_u64(RS& st, unsigned long long mn, unsigned long long mx) {
  if (threadIdx.x == 0) {
    st.kmin = ~0ull;
    st.kmax = 0ull;
  }
  bar();
  mn = wave_min_u64(mn);
  mx = wave_max_u64(mx);
  if (lane_id() == 0) {
    atomicMin(&st.kmin, mn);
    atomicMax(&st.kmax, mx);
  }
  bar();
}

// Staged block layout: token l at word l + l / 16, so that a thread reading its 16 consecutive tokens (word 17 t + k)
// and the other lanes of its wave hit distinct LDS banks.
constexpr int BIGW = BLK + BLK / 16;
__device__ inline int big_at(int l) { return l + (l >> 4); }

// A block's raw values as the stager loads them: the logits (thread layout of Blk), the mask words and the patches.
template <int DT>
struct Staged {
  using BL = Blk<DT, NT2>;
  float x[BL::EPT];
  uint32_t mw[BL::S];
  uint2 pv[TCAP / NT2];
  int lo, hi;  // the block's tokens
};
// Issues the loads of block g (recorded patches: n_patch >= 0) into S without waiting for them.
template <int DT>
__device__ __forceinline__ void stage_issue(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int g, Staged<DT>& S) {
  using BL = Blk<DT, NT2>;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  const int np = L.bi[g].n_patch;
  const QWS_G unsigned long long* PT = gmem((const unsigned long long*)(rec_of(ws, L.st->G, row, g) + PATCH_OFF));
#pragma unroll
  for (int k = 0; k < TCAP / NT2; k++) {
    const int p = (int)threadIdx.x + k * NT2;
    const unsigned long long w = p < np ? PT[p] : 0xFFFFFFFFull;  // {local index, value bits}; local ~0: none
    S.pv[k] = make_uint2((uint32_t)w, (uint32_t)(w >> 32));
  }
  BL::load_raw(B, row, lo, hi, S.x);
  BL::mask_words(B, R, lo, hi, S.mw);
  S.lo = lo;
  S.hi = hi;
}
// Block g from S into L.big in token order: NaN -> -inf, the mask, then the patches.  All threads; ends with a barrier.
template <int DT>
__device__ __forceinline__ void stage_store(const RL& L, const qws_row& R, int g, Staged<DT>& S) {
  using BL = Blk<DT, NT2>;
  float* xs = (float*)L.big;
  BL::fixnan(S.x);
  BL::apply_mask(R, S.lo, S.hi, S.mw, S.x);
#pragma unroll
  for (int e = 0; e < BL::EPT; e++) xs[big_at(BL::local(e))] = S.x[e];
  if (L.bi[g].n_patch > 0) {
    bar();
#pragma unroll
    for (int k = 0; k < TCAP / NT2; k++)
      if (S.pv[k].x != 0xFFFFFFFFu) xs[big_at((int)S.pv[k].x)] = __uint_as_float(S.pv[k].y);
  }
  bar();
}

// Block g of the row, processed, into L.big in token order (tokens past V read -inf).  With the block's patches
// recorded by k_scan the raw logits get the mask and the patches (the patches load together with the logits);
// otherwise the processors are rebuilt from the row's lists.  B and R are the workgroup's LDS copies.  All threads;
// ends with a barrier.
template <int DT>
__device__ __forceinline__ void stage_block_body(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int g) {
  using BL = Blk<DT, NT2>;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  if (R.proc_on && L.bi[g].n_patch < 0) {
    float x[BL::EPT];
    float* xs = (float*)L.big;
    load_processed<DT, NT2>(B, R, row, lo, hi, L.big, x, nullptr, L.nt);
    bar();
#pragma unroll
    for (int e = 0; e < BL::EPT; e++) xs[big_at(BL::local(e))] = x[e];
    bar();
    return;
  }
  Staged<DT> S;
  stage_issue<DT>(L, B, R, ws, row, g, S);
  stage_store<DT>(L, R, g, S);
}
// The out-of-line copy for the rare rescans (the draw stages its block inline: a call would spill the caller's
// registers to scratch around it).
template <int DT>
__device__ __noinline__ void stage_block(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int g) {
  stage_block_body<DT>(L, B, R, ws, row, g);
}

// The fine bins of row power p of every block into L.fb and summed over the row into st.fcnt / st.fmu.  Bins a block
// did not write lie below its deepest possible cut and read as empty.  Thread t loads fine bin t % 64 of blocks t / 64,
// t / 64 + 8, ... and sums them in registers; each wave's sums go to its row of st.part, and every wave then adds the
// eight rows up and writes the same totals (so no barrier is needed before a wave reads them).  All threads; when it
// stages, it begins with a barrier (the previous power's staged bins and sums may still be read) and has one more.
__device__ __forceinline__ void stage_power(const RL& L, char* ws, int row, int p) {
  RS& st = *L.st;
  const int G = st.G;
  if (st.fpow == p) return;  // uniform: every wave writes st.fpow itself, after the same barriers
  constexpr int NB = (MAXG * FB) / NT2;  // blocks per thread
  const int f = (int)threadIdx.x & 63, g0 = (int)threadIdx.x >> 6;
  unsigned long long w[NB];  // every load issued before the barrier
#pragma unroll
  for (int k = 0; k < NB; k++) {
    const int g = g0 + k * (NT2 / 64);
    w[k] = 0;
    if (g < G) {
      const BI& b = L.bi[g];
      const int pb = p - b.dn, rel = pb * FB + f;
      if (b.dn >= 0 && pb >= 0 && pb < NEXP && rel < b.nbw) w[k] = bins_of(ws, G, row, g)[rel];
    }
  }
  bar();
  uint32_t cn = 0;
  unsigned long long mu = 0;
#pragma unroll
  for (int k = 0; k < NB; k++) {
    const int g = g0 + k * (NT2 / 64);
    if (g < G) L.fb[g * FB + f] = w[k];
    cn += bw_cnt(w[k]);
    mu += bw_mu(w[k]);
  }
  st.pcnt[g0][f] = cn;
  st.pmu[g0][f] = mu;
  bar();
  cn = 0;
  mu = 0;
#pragma unroll
  for (int v = 0; v < NWV2; v++) {
    cn += st.pcnt[v][f];
    mu += st.pmu[v][f];
  }
  st.fcnt[f] = cn;  // every wave writes the same totals
  st.fmu[f] = mu;
  st.fpow = p;
}

// The first row power of two whose inclusive cumulative count reaches tgt (NEXP: none) -> *p, the count before it ->
// *before.  Every wave computes it from st.Rc (final after the per-power sums): no barrier.
__device__ __forceinline__ void pow_cross_cnt(const RL& L, unsigned long long tgt, int* p, unsigned long long* before) {
  const RS& st = *L.st;
  const int lane = lane_id();
  const unsigned long long v = lane < NEXP ? st.Rc[lane] : 0ull;
  const unsigned long long inc = wave_scan_incl<unsigned long long>(v);
  const int q = first_lane(lane < NEXP && inc >= tgt);
  const unsigned long long bf = readlane<unsigned long long>(inc - v, q < 64 ? q : 0);
  *p = q < NEXP ? q : NEXP;
  *before = q < NEXP ? bf : 0ull;
}
// The first row power whose inclusive cumulative mass (row units) reaches tgt (NEXP: none) -> *p, the mass before it
// -> *before.  Every wave, from st.Rm: no barrier.
__device__ __forceinline__ void pow_cross_mass(const RL& L, u128 tgt, int* p, u128* before) {
  const RS& st = *L.st;
  const int lane = lane_id();
  const u128 v = lane < NEXP ? shl128(st.Rm[lane], D_EXP - lane) : (u128)0;
  const u128 inc = wave_scan_incl_u128(v);
  const int q = first_lane(lane < NEXP && inc >= tgt);
  *before = readlane<u128>(inc - v, q < 64 ? q : 0);
  *p = q < NEXP ? q : NEXP;
}
// Over the staged power's fine bins: the first whose base + inclusive cumulative count (by_mass: mass in row units)
// reaches tgt -> returned (64: none), the cumulative value before it -> *before.  Every wave, from st.fcnt / st.fmu
// (final after stage_power): no barrier.
__device__ __forceinline__ int fine_cross(const RL& L, bool by_mass, u128 base, u128 tgt, u128* before) {
  const RS& st = *L.st;
  const int lane = lane_id();
  const u128 v = by_mass ? shl128(st.fmu[lane], D_EXP - st.fpow) : (u128)st.fcnt[lane];
  const u128 inc = wave_scan_incl_u128(v) + base;
  const int f = first_lane(inc >= tgt);
  *before = readlane<u128>(inc - v, f < 64 ? f : 0);
  return f;
}
// Mass (row units) and count of the row's candidates in bins above row bin r (r >= NR: every bin; else r's power's
// fine bins are staged).  Every wave, from st.Rm / st.Rc and the staged sums; ends with a barrier (the stage that
// follows may rewrite row state, such as the gathered bin's, that the stage before it read).
__device__ __forceinline__ void before_bin(const RL& L, int r, u128* mass, unsigned long long* count) {
  const RS& st = *L.st;
  const int lane = lane_id(), p = r >> 6;
  u128 m = lane < NEXP && lane < p ? shl128(st.Rm[lane], D_EXP - lane) : (u128)0;
  unsigned long long n = lane < NEXP && lane < p ? st.Rc[lane] : 0ull;
  if (r < NR && lane < (r & 63)) {
    m += shl128(st.fmu[lane], D_EXP - p);
    n += st.fcnt[lane];
  }
  *mass = wave_sum_u128(m);
  *count = wave_sum<unsigned long long>(n);
  bar();
}

// The smallest value x, in the order -inf < ... < -0 < +0 < ... < +inf, with tval(x, K) >= tc (tval is monotone in
// x, so tval(x, K) >= tc  <=>  x >= that value  <=>  okey(x) >= its okey).  From tc / K in a few steps of one value;
// false if more than 64 steps would be needed (the caller then selects by count).
__device__ inline bool first_x_t(float tc, float K, float* out) {
  if (tval(-INFINITY, K) >= tc) {
    *out = -INFINITY;
    return true;
  }
  auto step = [](float v, int d) {  // the next value below (d = -1) or above (d = 1), -0 and +0 distinct
    const uint32_t u = __float_as_uint(v);
    return okey_val(((u & 0x80000000u) ? ~u : (u | 0x80000000u)) + (uint32_t)d);
  };
  float x = tc / K;
  if (!(x == x) || fabsf(x) == INFINITY) return false;
  int n = 0;
  while (tval(x, K) >= tc && n < 64) {
    x = step(x, -1);
    n++;
  }
  while (!(tval(x, K) >= tc) && n < 128) {
    x = step(x, 1);
    n++;
  }
  if (n >= 64 || !(tval(x, K) >= tc) || tval(step(x, -1), K) >= tc) return false;
  *out = x;
  return true;
}

// block of flat gathered-list index i (blocks' gofs ascending, list sources only)
__device__ inline int gblock_at(const RL& L, int G, int i) {
  int a = 0, b = G - 1;
  while (a < b) {
    const int m = (a + b + 1) >> 1;
    if (L.bi[m].gofs <= i)
      a = m;
    else
      b = m - 1;
  }
  return a;
}
__device__ inline uint32_t mu_of_comp(uint64_t c, float K, const float2* ts) { return weigh(tval(okey_val(comp_key(c)), K), ts).mu; }

// A value range that holds every x of row bin `qb` (floor(tval(x, K)) >> 4 == qb), for rescans that test the exact bin
// only for values inside it.  t = fl(x * K) in [16 qb, 16 qb + 16) puts the exact product x * K within half an ulp of
// that interval: within 1 below |t| < 2^24 and within 2^-24 |t| above, both inside the margins of 1 + 10^-5 |t| in t
// (the float rounding of the edges divided by K is smaller still).  A bin at the clamps of t (x * K at or beyond
// +-2^30) passes every value.
struct XRange {
  float lo, hi;
  __device__ inline bool maybe(float v) const { return v >= lo && v <= hi; }
};
__device__ inline XRange bin_xrange(int qb, float K) {
  const long long t0 = 16ll * qb;
  if (!(t0 > -(1ll << 30) + 16 && t0 + 32 < (1ll << 30))) return {-INFINITY, INFINITY};
  const double lo = (double)(t0 - 1) - fabs((double)t0) * 1e-5, hi = (double)(t0 + 17) + fabs((double)(t0 + 16)) * 1e-5;
  return {(float)(lo / (double)K), (float)(hi / (double)K)};
}

// Calls fn(comp, mu) for every candidate of row bin rb (gathered: from LDS; else from the blocks' lists and rescans).
// All threads; ends with a barrier.
template <int DT, typename F>
__device__ __forceinline__ void for_bin(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, F fn) {
  using BL = Blk<DT, NT2>;
  const RS& st = *L.st;
  const int tid = threadIdx.x;
  if (st.gstaged) {
    for (int i = tid; i < st.gn; i += NT2) fn(L.ec[i], L.em[i]);
    bar();
    return;
  }
  const int G = st.G, rb = st.gbin;
  for (int i = tid; i < st.gl; i += NT2) {
    const int g = gblock_at(L, G, i);
    const BI& b = L.bi[g];
    const uint64_t c = els_of(ws, G, row, g)[b.goff + (i - b.gofs)];
    fn(c, mu_of_comp(c, st.K, L.ts));
  }
  for (int g = 0; g < (st.gres ? G : 0); g++) {
    if (L.bi[g].gsrc != 2) continue;
    stage_block<DT>(L, B, R, ws, row, g);
    const float* xs = (const float*)L.big;
    const int t0 = tid * BL::EPT;
#pragma unroll
    for (int k = 0; k < BL::EPT; k++) {
      const float v = xs[big_at(t0) + k];
      const W w = weigh(tval(v, st.K), L.ts);
      if (v != -INFINITY && st.row_top - w.bin() == rb) fn(comp(okey(v), (uint32_t)(g * BLK + t0 + k)), w.mu);
    }
    bar();
  }
  bar();
}

// Gathers row bin rb (its power's fine bins staged): each block's elements come from its list when its window held
// the bin, else from a rescan of the block.  The bin is held in LDS when it has at most XG elements.  SKIP: a batch of
// rescans loads only its blocks (the verify rows' instance).  All threads.
template <int DT, bool SKIP>
__device__ __forceinline__ void gather(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int rb) {
  RS& st = *L.st;
  const int G = st.G, tid = threadIdx.x;
  if (st.gbin == rb) return;  // uniform: st.gbin is written only after the barrier below, which every wave passes after this test
  if (tid < 64) {
    // slots of the staged bin: the listed blocks' elements first (block order), then those of the blocks rescanned
    // from their raw logits (block order, each at a slot range fixed by its bin count), then the other rescans
    const int g = tid;
    uint32_t cn = 0, ln = 0, fr = 0;
    int nres = 0;
    if (g < G) {
      BI& b = L.bi[g];
      const unsigned long long w = L.fb[g * FB + (rb & 63)];
      cn = bw_cnt(w);
      b.gcnt = (int)cn;
      b.goff = (int)bw_off(w);
      b.gsrc = cn == 0 ? 0 : ((bw_listed(w) && !(R.test_flags & QWS_TF_RESCAN)) ? 1 : 2);
      ln = b.gsrc == 1 ? cn : 0u;
      fr = b.gsrc == 2 && !R.mask_mode && b.n_patch == 0 ? cn : 0u;
      nres = b.gsrc == 2 ? 1 : 0;
    }
    const uint32_t linc = wave_scan_incl<uint32_t>(ln), finc = wave_scan_incl<uint32_t>(fr);
    const uint32_t tot = wave_sum<uint32_t>(cn), nl = readlane<uint32_t>(linc, 63);
    const bool staged = tot <= (uint32_t)XG;
    const unsigned long long fast = staged ? __ballot(fr != 0) : 0ull, slow = __ballot(nres != 0) & ~fast;
    if (g < G) {
      // unstaged, gofs stays the listed prefix (ascending over the blocks, as for_bin's block search needs)
      L.bi[g].gofs = fr && staged ? (int)(nl + finc - fr) : (int)(linc - ln);
      if (fr && staged) L.bi[g].goff = 0;  // the rescan's slot cursor (a rescanned block has no list offset)
    }
    const int nr = wave_sum<int>(nres);
    if (tid == 0) {
      st.gl = (int)nl;
      st.gn = (int)tot;
      st.gstaged = 0;
      st.gres = nr;
      st.gfast = fast;
      st.gslow = slow;
      st.gmin = ~0ull;  // the staged bin's comp range, reduced by one atomic per wave at the end
      st.gmax = 0ull;
      st.si[7] = (int)(nl + readlane<uint32_t>(finc, 63));  // the first slot of the other rescans
      st.rescans += nr;
    }
  }
  bar();
  if (tid == 0) st.gbin = rb;  // read again only after this function's last barrier
  if (st.gn <= XG) {
    const int nl = st.gl;
    // eight threads per block (G <= 64), each loading every eighth element of its block's list range, U loads in
    // flight (a block's first 64 elements in one round); the comp range of the bin is reduced on the way (the
    // selection's first range)
    constexpr int U = 8;
    unsigned long long mn = ~0ull, mx = 0ull;
    {
      const int g = tid >> 3, j = tid & 7;
      if (g < G && L.bi[g].gsrc == 1) {
        const BI& b = L.bi[g];
        const QWS_G uint64_t* src = els_of(ws, G, row, g) + b.goff;
        for (int i0 = j; i0 < b.gcnt; i0 += 8 * U) {
          uint64_t cv[U];
#pragma unroll
          for (int k = 0; k < U; k++) cv[k] = i0 + 8 * k < b.gcnt ? src[i0 + 8 * k] : 0ull;
#pragma unroll
          for (int k = 0; k < U; k++) {
            const int i = i0 + 8 * k;
            if (i < b.gcnt) {
              L.ec[b.gofs + i] = cv[k];
              L.em[b.gofs + i] = mu_of_comp(cv[k], st.K, L.ts);
              mn = cv[k] < mn ? cv[k] : mn;
              mx = cv[k] > mx ? cv[k] : mx;
            }
          }
        }
      }
    }
    bar();
    using BL = Blk<DT, NT2>;
    {
      // blocks without processed tokens or a mask: their raw logits are their values, read straight into registers,
      // RB blocks at once (all their loads in flight together); only the bin's elements are weighed, each placed at its
      // block's next slot
      constexpr int RB = 8;  // the resolver runs one workgroup per CU: registers for eight blocks of loads in flight
      const int qb = st.row_top - rb;  // the bin's floor(t) >> 4
      const float K = st.K;
      const XRange xr = bin_xrange(qb, K);
      unsigned long long fm = st.gfast;  // uniform
      while (fm) {
        int gb[RB];
#pragma unroll
        for (int k = 0; k < RB; k++) {
          gb[k] = fm ? __ffsll((long long)fm) - 1 : -1;
          fm &= fm - 1ull;
        }
        // every load issued before any is used.  SKIP (the verify rows' instance): an unused slot loads nothing, since
        // one CU reads a block at ~16 bytes per cycle; the sampling rows' instance reads the first block again there
        // instead (no branch around the loads: the skipping code slowed that kernel's other paths by its layout)
        float x[RB][BL::EPT];
#pragma unroll
        for (int k = 0; k < RB; k++) {
          if constexpr (SKIP) {
            if (gb[k] >= 0) BL::load_raw(B, row, gb[k] * BLK, min(B.V, gb[k] * BLK + BLK), x[k]);  // uniform; -inf past V
          } else {
            const int gk = gb[k] >= 0 ? gb[k] : gb[0];
            BL::load_raw(B, row, gk * BLK, min(B.V, gk * BLK + BLK), x[k]);  // -inf past V; NaN tested below
          }
        }
#pragma unroll
        for (int k = 0; k < RB; k++) {
          if (gb[k] < 0) continue;
          BI& b = L.bi[gb[k]];
#pragma unroll
          for (int e = 0; e < BL::EPT; e++) {
            const float v = x[k][e];
            if (!xr.maybe(v)) continue;  // NaN fails it too
            const float t = tval(v, K);
            if (v == v && v != -INFINITY && (tfloor(t) >> 4) == qb) {  // NaN counts as -inf
              const int p = b.gofs + atomicAdd(&b.goff, 1);
              const uint64_t c = comp(okey(v), (uint32_t)(gb[k] * BLK + BL::local(e)));
              mn = c < mn ? c : mn;
              mx = c > mx ? c : mx;
              if (p < XG) {  // always: the bin words count these elements
                L.ec[p] = c;
                L.em[p] = weigh(t, L.ts).mu;
              }
            }
          }
        }
      }
    }
    for (unsigned long long sm = st.gslow; sm; sm &= sm - 1ull) {  // uniform: read after the barrier
      const int g = __ffsll((long long)sm) - 1;
      if (tid == 0) L.bi[g].gofs = st.si[7];  // the block's elements follow (their order within the block is free)
      stage_block<DT>(L, B, R, ws, row, g);
      const float* xs = (const float*)L.big;
      const int t0 = tid * BL::EPT;
#pragma unroll
      for (int k = 0; k < BL::EPT; k++) {
        const float v = xs[big_at(t0) + k];
        const W w = weigh(tval(v, st.K), L.ts);
        if (v != -INFINITY && st.row_top - w.bin() == rb) {
          const int p = atomicAdd(&st.si[7], 1);
          const uint64_t c = comp(okey(v), (uint32_t)(g * BLK + t0 + k));
          mn = c < mn ? c : mn;
          mx = c > mx ? c : mx;
          if (p < XG) {  // always: the bin words count these elements
            L.ec[p] = c;
            L.em[p] = w.mu;
          }
        }
      }
      bar();
    }
    mn = wave_min_u64(mn);
    mx = wave_max_u64(mx);
    if (lane_id() == 0) {
      atomicMin(&st.gmin, mn);
      atomicMax(&st.gmax, mx);
    }
    if (tid == 0) st.gstaged = 1;
  }
  bar();
}

// The selection: in comp-descending order over the gathered bin, the first element whose inclusive prefix of value
// (1 per element, or its mantissa) reaches target (>= 1): its comp -> st.su[4] and that prefix -> st.su[5] (both
// left as they were when the target exceeds the bin's total).  Radix refinement on the whole comp (value key, then
// index): each round buckets the elements of the current comp range into NBK equal ranges, finds the bucket where the
// prefix crosses the target and narrows the range to it; at most a wave of elements left are ranked directly.
//
// select_rounds: the rounds from the comp range [kmin, kmax] with value base before it.  All threads, after a barrier
// that follows the last reads of the buckets.
template <int DT>
__device__ __forceinline__ void select_rounds(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, bool by_mass, uint64_t target,
                                              uint64_t kmin, uint64_t kmax, uint64_t base) {
  RS& st = *L.st;
  const int tid = threadIdx.x;
  for (int round = 0; round < 16; round++) {
    const int sh = bucket_shift(kmax - kmin);
    for (int i = tid; i < NBK; i += NT2) {
      st.bcnt[i] = 0;
      st.bsum[i] = 0;
    }
    bar();
    for_bin<DT>(L, B, R, ws, row, [&](uint64_t c, uint32_t mu) {
      if (c >= kmin && c <= kmax) {
        const int b = NBK - 1 - (int)((c - kmin) >> sh);  // bucket 0 = the largest comps
        atomicAdd(&st.bcnt[b], 1u);
        atomicAdd(&st.bsum[b], by_mass ? (unsigned long long)mu : 1ull);
      }
    });
    if (wave_id() == 0) {  // the bucket where base + the prefix of the bucket values crosses the target
      const int lane = lane_id();
      uint64_t v[NBK / 64], loc = 0;
#pragma unroll
      for (int k = 0; k < NBK / 64; k++) {
        v[k] = st.bsum[lane * (NBK / 64) + k];
        loc += v[k];
      }
      const uint64_t incl = wave_scan_incl<uint64_t>(loc);
      uint64_t run = base + incl - loc, before = 0;
      int hit = -1;
#pragma unroll
      for (int k = 0; k < NBK / 64; k++) {
        if (hit < 0 && run + v[k] >= target) {
          hit = lane * (NBK / 64) + k;
          before = run;
        }
        run += v[k];
      }
      const int l = first_lane(hit >= 0);
      if (lane == (l < 64 ? l : 0)) {
        st.si[4] = l < 64 ? hit : -1;
        st.su[6] = before;
        st.si[5] = l < 64 ? (int)st.bcnt[hit] : 0;
      }
    }
    bar();
    const int hb = st.si[4];
    if (hb < 0) return;  // the target exceeds the total
    base = st.su[6];
    const int nb = st.si[5];
    const uint64_t bl = kmin + ((uint64_t)(NBK - 1 - hb) << sh);
    const uint64_t span = (1ull << sh) - 1;
    const uint64_t bh = kmax - bl <= span ? kmax : bl + span;
    if (nb <= 64) {  // at most a wave of elements left: wave 0 ranks them directly
      if (tid == 0) st.si[3] = 0;
      bar();
      for_bin<DT>(L, B, R, ws, row, [&](uint64_t c, uint32_t mu) {
        if (c >= bl && c <= bh) {
          const int p = atomicAdd(&st.si[3], 1);
          if (p < 64) {  // always: the bucket held nb <= 64 of them
            st.xs[p] = c;
            st.xv[p] = by_mass ? (uint64_t)mu : 1ull;
          }
        }
      });
      if (wave_id() == 0) {
        const int lane = lane_id();
        const uint64_t c = lane < nb ? st.xs[lane] : 0ull;
        const uint64_t v = lane < nb ? st.xv[lane] : 0ull;
        uint64_t above = 0;  // value of the elements with a larger comp
        for (int j = 0; j < nb; j++) {
          const uint64_t cj = readlane<uint64_t>(c, j), vj = readlane<uint64_t>(v, j);
          above += cj > c ? vj : 0ull;
        }
        const bool hit = lane < nb && base + above < target && base + above + v >= target;
        const int l = first_lane(hit);
        if (lane == (l < 64 ? l : 0) && l < 64) {
          st.su[4] = c;
          st.su[5] = base + above + v;
        }
      }
      bar();
      return;
    }
    kmin = bl;
    kmax = bh;
  }
}
// select_in_bin: the selection over the gathered bin (gather called first).  All threads.
template <int DT>
__device__ __forceinline__ void select_in_bin(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, bool by_mass, uint64_t target) {
  RS& st = *L.st;
  if (!st.gstaged) {
    unsigned long long mn = ~0ull, mx = 0ull;
    for_bin<DT>(L, B, R, ws, row, [&](uint64_t c, uint32_t) {
      mn = c < mn ? c : mn;
      mx = c > mx ? c : mx;
    });
    block_range_u64(st, mn, mx);
  } else {
    bar();
  }
  const uint64_t kmin = st.gstaged ? st.gmin : st.kmin, kmax = st.gstaged ? st.gmax : st.kmax;
  if (kmin > kmax) return;
  select_rounds<DT>(L, B, R, ws, row, by_mass, target, kmin, kmax, 0ull);
}

// The gather and selection of row bin rb together, for a bin whose elements all lie in their blocks' lists and fit
// in LDS (the dense cut bin of a flat row): every wave finds each element's block from the per-block counts held in
// its lanes, so the element loads need no barrier before them; the first bucket round runs over the elements held in
// registers; every wave finds the crossing bucket and ranks its elements itself.  Three barriers where gather and
// select_in_bin take about ten; the same result, and the same gathered-bin state left in LDS.  The crossing
// element's comp -> *cut, its inclusive prefix -> *incl (~0 and 0 when the target exceeds the bin's total).  Returns
// false, having changed nothing, when the bin does not qualify (a block's elements not listed, more than XG
// elements, rescans or separate passes asked for by the test flags, or the bin gathered already).  A barrier must
// separate the previous selection's last reads of its buckets from this call.  All threads.
constexpr int XS = XG / NT2;  // elements per thread
static_assert(XG % NT2 == 0 && MAXG <= 64, "select_listed layout");
template <int DT>
__device__ __forceinline__ bool select_listed(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int rb, bool by_mass, uint64_t target,
                                              uint64_t* cut, uint64_t* incl) {
  RS& st = *L.st;
  const int G = st.G, tid = threadIdx.x, lane = lane_id();
  if (st.gbin == rb || (R.test_flags & (QWS_TF_RESCAN | QWS_TF_SPLIT_SELECT))) return false;  // uniform: st.gbin is written after the first barrier below
  uint32_t cn = 0, off = 0;  // lane g: block g's count in the bin and its list offset
  bool unlisted = false;
  if (lane < G) {
    const unsigned long long w = L.fb[lane * FB + (rb & 63)];
    cn = bw_cnt(w);
    off = bw_off(w);
    unlisted = cn != 0 && !bw_listed(w);
  }
  const uint32_t inc = wave_scan_incl<uint32_t>(cn), tot = readlane<uint32_t>(inc, 63), exc = inc - cn;
  if (__ballot(unlisted) != 0ull || tot == 0u || tot > (uint32_t)XG) return false;  // uniform: the same words in every wave
  if (tid < 64) {  // the gathered-bin state gather leaves: block g's elements at LDS slots [exc, inc)
    if (lane < G) {
      BI& b = L.bi[lane];
      b.gcnt = (int)cn;
      b.goff = (int)off;
      b.gsrc = cn ? 1 : 0;
      b.gofs = (int)exc;
    }
    if (lane == 0) {
      st.gl = st.gn = (int)tot;
      st.gstaged = 1;
      st.gres = 0;
      st.gfast = st.gslow = 0ull;
      st.si[3] = 0;
    }
  }
  for (int i = tid; i < NBK; i += NT2) {
    st.bcnt[i] = 0u;
    st.bsum[i] = 0ull;
  }
  // element i = tid + k NT2 of the bin (blocks in order, each block's in list order): its block by a binary search
  // over the lanes' inclusive counts; every load issued before any is used (a slot past the end reloads the last)
  uint64_t ce[XS];
  uint32_t me[XS];
#pragma unroll
  for (int k = 0; k < XS; k++) {
    if (k * NT2 >= (int)tot) break;  // uniform
    const int i = min(tid + k * NT2, (int)tot - 1);
    int g = 0;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) g += __shfl((int)inc, g + s - 1) <= i ? s : 0;
    const int e = __shfl((int)exc, g), o = __shfl((int)off, g);
    ce[k] = els_of(ws, G, row, g)[o + (i - e)];
  }
  unsigned long long mn = ~0ull, mx = 0ull;
#pragma unroll
  for (int k = 0; k < XS; k++) {
    if (k * NT2 >= (int)tot) break;  // uniform
    const int i = tid + k * NT2;
    me[k] = mu_of_comp(ce[k], st.K, L.ts);
    if (i < (int)tot) {
      L.ec[i] = ce[k];
      L.em[i] = me[k];
      mn = ce[k] < mn ? ce[k] : mn;
      mx = ce[k] > mx ? ce[k] : mx;
    }
  }
  mn = wave_min_u64(mn);
  mx = wave_max_u64(mx);
  if (lane == 0) {
    st.wmn[wave_id()] = mn;
    st.wmx[wave_id()] = mx;
  }
  bar();
  if (tid == 0) st.gbin = rb;
  uint64_t kmin = st.wmn[0], kmax = st.wmx[0];
#pragma unroll
  for (int w = 1; w < NWV2; w++) {
    kmin = st.wmn[w] < kmin ? st.wmn[w] : kmin;
    kmax = st.wmx[w] > kmax ? st.wmx[w] : kmax;
  }
  if (tid == 0) {  // the bin's range, as gather leaves it
    st.gmin = kmin;
    st.gmax = kmax;
  }
  const int sh = bucket_shift(kmax - kmin);
#pragma unroll
  for (int k = 0; k < XS; k++) {
    if (k * NT2 >= (int)tot) break;  // uniform
    if (tid + k * NT2 < (int)tot) {
      const int b = NBK - 1 - (int)((ce[k] - kmin) >> sh);  // bucket 0 = the largest comps
      atomicAdd(&st.bcnt[b], 1u);
      atomicAdd(&st.bsum[b], by_mass ? (unsigned long long)me[k] : 1ull);
    }
  }
  bar();
  // every wave: the bucket where the prefix of the bucket values crosses the target
  uint64_t base;
  int hb, nb;
  {
    uint64_t v[NBK / 64], loc = 0;
#pragma unroll
    for (int k = 0; k < NBK / 64; k++) {
      v[k] = st.bsum[lane * (NBK / 64) + k];
      loc += v[k];
    }
    const uint64_t inc2 = wave_scan_incl<uint64_t>(loc);
    uint64_t run = inc2 - loc, before = 0;
    int hit = -1;
#pragma unroll
    for (int k = 0; k < NBK / 64; k++) {
      if (hit < 0 && run + v[k] >= target) {
        hit = lane * (NBK / 64) + k;
        before = run;
      }
      run += v[k];
    }
    const int l = first_lane(hit >= 0);
    if (l >= 64) {  // the target exceeds the bin's total
      *cut = ~0ull;
      *incl = 0ull;
      return true;
    }
    hb = readlane<int>(hit, l);
    base = readlane<uint64_t>(before, l);
    nb = (int)st.bcnt[hb];
  }
  const uint64_t bl = kmin + ((uint64_t)(NBK - 1 - hb) << sh);
  const uint64_t span = (1ull << sh) - 1;
  const uint64_t bh = kmax - bl <= span ? kmax : bl + span;
  if (nb > 64) {  // more rounds, over the elements in LDS
    bar();
    select_rounds<DT>(L, B, R, ws, row, by_mass, target, bl, bh, base);
    *cut = st.su[4];
    *incl = st.su[5];
    return true;
  }
#pragma unroll
  for (int k = 0; k < XS; k++) {
    if (k * NT2 >= (int)tot) break;  // uniform
    if (tid + k * NT2 < (int)tot && ce[k] >= bl && ce[k] <= bh) {
      const int p = atomicAdd(&st.si[3], 1);
      if (p < 64) {  // always: the bucket holds nb <= 64 of them
        st.xs[p] = ce[k];
        st.xv[p] = by_mass ? (uint64_t)me[k] : 1ull;
      }
    }
  }
  bar();
  // every wave: the bucket's elements ranked directly
  const uint64_t c = lane < nb ? st.xs[lane] : 0ull;
  const uint64_t v = lane < nb ? st.xv[lane] : 0ull;
  uint64_t above = 0;  // value of the elements with a larger comp
  for (int j = 0; j < nb; j++) {  // uniform
    const uint64_t cj = readlane<uint64_t>(c, j), vj = readlane<uint64_t>(v, j);
    above += cj > c ? vj : 0ull;
  }
  const int l = first_lane(lane < nb && base + above < target && base + above + v >= target);
  *cut = l < 64 ? readlane<uint64_t>(c, l) : ~0ull;
  *incl = l < 64 ? base + readlane<uint64_t>(above + v, l) : 0ull;
  return true;
}

// The top-p cut inside row bin rb together with every block's kept mass, for a bin whose elements every block holding
// some has listed (at most 8 FPT per block): the common case of a flat row's dense cut bin.  Eight threads per block
// each load up to FPT of the block's listed elements of rb into registers and weigh them; the elements are bucketed by
// their value key over the key range the bin's t interval [16 qb, 16 qb + 16) spans (clamped at its ends, so the
// buckets stay in comp order without a reduction of the actual range); every wave finds the bucket where the prefix
// of the mantissas (comp-descending) crosses target, and ranks that bucket's elements (at most 64) itself.  Then the
// same eight threads of each block sum its kept mass in row units -- its powers above the cut's, its fine bins above
// rb and its elements of rb from the cut on -- into st.Klo / st.Khi.  Three barriers where select_listed and the
// separate kept-mass pass take about seven.  The crossing element's comp -> *cut, its inclusive mantissa prefix ->
// *incl.  Returns false, having changed nothing the other paths read, when the bin does not qualify (a block's
// elements not listed or more than 8 FPT of them, the bin gathered already, test flags asking for other paths) or
// its crossing bucket holds more than 64 elements.  rb's power must be the staged one, and the fast-cut state
// (st.fbc, st.fbs, st.fxn) as k_resolve's start leaves it.  All threads; ends with a barrier.
constexpr int FPT = 8;
static_assert(MAXG * 8 <= NT2, "eight threads per block");
__device__ __forceinline__ bool topp_cut_fast(const RL& L, const qws_row& R, char* ws, int row, int rb, uint64_t target, uint64_t* cut,
                                              uint64_t* incl) {
  RS& st = *L.st;
  const int G = st.G, tid = threadIdx.x, lane = lane_id();
  if (st.gbin == rb || (R.test_flags & (QWS_TF_RESCAN | QWS_TF_SPLIT_SELECT))) return false;  // uniform
  {
    bool bad = false;
    if (lane < G) {
      const unsigned long long w = L.fb[lane * FB + (rb & 63)];
      const uint32_t cn = bw_cnt(w);
      bad = cn != 0 && (!bw_listed(w) || cn > 8u * FPT);
    }
    if (__ballot(bad) != 0ull) return false;  // uniform: the same words in every wave
  }
  const int g = tid >> 3, j = tid & 7;
  const bool own = g < G;
  uint32_t cn = 0, off = 0;
  if (own) {
    const unsigned long long w = L.fb[g * FB + (rb & 63)];
    cn = bw_cnt(w);
    off = bw_off(w);
  }
  // the block's elements j, j + 8, ...: every load issued before any is used
  uint64_t ce[FPT];
  uint32_t me[FPT];
  {
    const QWS_G uint64_t* src = els_of(ws, G, row, own ? g : 0) + off;
#pragma unroll
    for (int k = 0; k < FPT; k++) ce[k] = j + 8 * k < (int)cn ? src[j + 8 * k] : 0ull;
  }
  // each block's kept mass above the cut bin in row units, while the loads are in flight: its powers above the cut's
  // (u128) and its fine bins above rb (mantissas, < 2^40 for eight of them), summed over the block's eight lanes
  const int pc = rb >> 6, fsh = D_EXP - pc;
  u128 km = 0;
  uint64_t mbin = 0;
  if (own && L.bi[g].dn >= 0) {
    const int dn = L.bi[g].dn;
    for (int er = dn + j; er < pc; er += 8) km += shl128(L.emu[g * NEXP + er - dn], D_EXP - er);
    for (int f = j; f < (rb & 63); f += 8) mbin += bw_mu(L.fb[g * FB + f]);
  }
#pragma unroll
  for (int x = 1; x < 8; x <<= 1) {  // sums over the block's eight lanes (xor partners stay inside the group)
    uint32_t w[6] = {(uint32_t)km, (uint32_t)(km >> 32), (uint32_t)(km >> 64), (uint32_t)(km >> 96), (uint32_t)mbin, (uint32_t)(mbin >> 32)};
#pragma unroll
    for (int i = 0; i < 6; i++) w[i] = (uint32_t)__shfl_xor((int)w[i], x);
    km += ((u128)w[3] << 96) | ((u128)w[2] << 64) | ((u128)w[1] << 32) | (u128)w[0];
    mbin += ((uint64_t)w[5] << 32) | w[4];
  }
  // bucket range: the keys of the bin's t interval (x = t / K is increasing in t for K > 0)
  const float K = st.K;
  const int qb = st.row_top - rb;
  const uint32_t klo = okey((float)(16 * qb) / K), khi = okey((float)(16 * qb + 16) / K);
  const uint32_t span = khi > klo ? khi - klo : 0u;
  const int bsh = max((span ? 32 - __clz((int)span) : 0) - 8, 0);
#pragma unroll
  for (int k = 0; k < FPT; k++) {
    if (j + 8 * k >= (int)cn) continue;
    me[k] = mu_of_comp(ce[k], K, L.ts);
    const uint32_t key = comp_key(ce[k]);
    const uint32_t d = key > klo ? (key - klo) >> bsh : 0u;
    const int b = NBK - 1 - (int)min(d, (uint32_t)(NBK - 1));  // bucket 0 = the largest keys
    atomicAdd(&st.fbc[b], 1u);
    atomicAdd(&st.fbs[b], (unsigned long long)me[k]);
  }
  bar();
  // every wave: the bucket where the prefix of the bucket sums crosses the target
  uint64_t base;
  int hb, nb;
  {
    uint64_t v[NBK / 64], loc = 0;
#pragma unroll
    for (int k = 0; k < NBK / 64; k++) {
      v[k] = st.fbs[lane * (NBK / 64) + k];
      loc += v[k];
    }
    const uint64_t inc2 = wave_scan_incl<uint64_t>(loc);
    uint64_t run = inc2 - loc, before = 0;
    int hit = -1;
#pragma unroll
    for (int k = 0; k < NBK / 64; k++) {
      if (hit < 0 && run + v[k] >= target) {
        hit = lane * (NBK / 64) + k;
        before = run;
      }
      run += v[k];
    }
    const int l = first_lane(hit >= 0);
    if (l >= 64) return false;  // uniform: the target exceeds the bin (not reached: the bin was found by this target)
    hb = readlane<int>(hit, l);
    base = readlane<uint64_t>(before, l);
    nb = (int)st.fbc[hb];
  }
  if (nb > 64) return false;  // uniform
  {
#pragma unroll
    for (int k = 0; k < FPT; k++) {
      if (j + 8 * k >= (int)cn) continue;
      const uint32_t key = comp_key(ce[k]);
      const uint32_t d = key > klo ? (key - klo) >> bsh : 0u;
      if (NBK - 1 - (int)min(d, (uint32_t)(NBK - 1)) == hb) {
        const int p = atomicAdd(&st.fxn, 1);
        if (p < 64) {  // always: the bucket holds nb <= 64 of them
          st.fxs[p] = ce[k];
          st.fxv[p] = me[k];
        }
      }
    }
  }
  bar();
  // every wave: the bucket's elements ranked directly
  uint64_t cC, pref;
  {
    const uint64_t c = lane < nb ? st.fxs[lane] : 0ull;
    const uint64_t v = lane < nb ? st.fxv[lane] : 0ull;
    uint64_t above = 0;  // value of the elements with a larger comp
    for (int i = 0; i < nb; i++) {  // uniform
      const uint64_t ci = readlane<uint64_t>(c, i), vi = readlane<uint64_t>(v, i);
      above += ci > c ? vi : 0ull;
    }
    const int l = first_lane(lane < nb && base + above < target && base + above + v >= target);
    if (l >= 64) return false;  // uniform (not reached: the bucket holds the crossing)
    cC = readlane<uint64_t>(c, l);
    pref = base + readlane<uint64_t>(above + v, l);
  }
  // each block's kept elements of rb (mantissas), summed over its eight lanes, complete its kept mass
  uint64_t mown = 0;
#pragma unroll
  for (int k = 0; k < FPT; k++)
    if (j + 8 * k < (int)cn && ce[k] >= cC) mown += me[k];
#pragma unroll
  for (int x = 1; x < 8; x <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)mown, x), hi = (uint32_t)__shfl_xor((int)(uint32_t)(mown >> 32), x);
    mown += ((uint64_t)hi << 32) | lo;
  }
  km += shl128(mbin + mown, fsh);
  if (own && j == 0) {
    st.Klo[g] = (unsigned long long)km;
    st.Khi[g] = (unsigned long long)(km >> 64);
  }
  bar();
  *cut = cC;
  *incl = pref;
  return true;
}

// The draw inside block g when its kept set lies whole in its list (every bin down to the cut listed, n <= 64 listed
// elements there): the token whose interval of the kept weights (index order) holds the local target tl, from lane i
// holding listed element i.  One wave; the same token as draw_in_block.
__device__ __forceinline__ int draw_listed(const RL& L, char* ws, int row, int g, int n, int cR, uint64_t cC, u128 tl) {
  const RS& st = *L.st;
  const int lane = lane_id();
  uint64_t w = 0;
  uint32_t idx = 0xFFFFFFFFu;
  if (lane < n) {
    const uint64_t c = els_of(ws, st.G, row, g)[lane];
    const float t = tval(okey_val(comp_key(c)), st.K);
    const int r = st.row_top - (tfloor(t) >> 4);
    if (r < cR || (r == cR && r < NR && c >= cC)) w = rw1(weigh(t, L.ts).mu, r);  // cR == NR: no cut
    idx = comp_idx(c);
  }
  u128 below = 0;  // kept weight of the listed elements before this one in index order
  for (int j = 0; j < n; j++) {  // uniform
    const uint32_t ij = readlane<uint32_t>(idx, j);
    const uint64_t wj = readlane<uint64_t>(w, j);
    below += ij < idx ? (u128)wj : (u128)0;
  }
  const int l = first_lane(w != 0 && below <= tl && tl < below + w);
  return l < 64 ? (int)readlane<uint32_t>(idx, l) : -1;
}

// Kept weight (row units) of one staged token: 0 outside the cut.  NINF: -inf excluded by value, needed when the row's
// best lies within the window's depth of the lower clamp (-inf shares t = -2^30 with the clamped finite values)
// t = tval(v, K) and e its table entry (read beforehand, so that no branch separates the loop's LDS reads)
template <bool NINF>
__device__ __forceinline__ uint64_t kept_weight(float v, float t, float2 e, int row_top, int cR, uint64_t cC, uint32_t idx) {
  const W ww = weigh_e(t, e);
  const int r = row_top - ww.bin();
  bool keep = r < cR;
  if (r == cR) keep = r < NR && comp(okey(v), idx) >= cC;  // cR == NR: no cut
  if constexpr (NINF) keep = keep && v != -INFINITY;
  const uint64_t wk = (uint64_t)ww.mu << (D_EXP - min(r >> 6, D_EXP));  // r >= 0: no token lies above the row's best
  return keep ? wk : 0ull;
}

// The token whose interval of the kept weights of block g (index order) holds the local target tl.  All threads.
template <int DT>
__device__ __forceinline__ int draw_in_block(const RL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int g, int cR, uint64_t cC, u128 tl) {
  using BL = Blk<DT, NT2>;
  constexpr int EPT = BL::EPT;
  RS& st = *L.st;
  const int lo = g * BLK;
  const float* xs = (const float*)L.big;
  if (threadIdx.x == 0) st.si[2] = -1;
  stage_block_body<DT>(L, B, R, ws, row, g);  // the processed block in L.big, token order
  const int t0 = (int)threadIdx.x * EPT;
  const float K = st.K;
  const int row_top = st.row_top;
  // the thread's values, then their table entries, each in one round of LDS reads
  float xv[EPT], tv[EPT];
  float2 te[EPT];
#pragma unroll
  for (int k = 0; k < EPT; k++) xv[k] = xs[big_at(t0) + k];
#pragma unroll
  for (int k = 0; k < EPT; k++) {
    tv[k] = tval(xv[k], K);
    te[k] = L.ts[tab_index(tv[k])];
  }
  uint64_t w[EPT];
  uint64_t loc = 0;  // EPT weights < 2^59 each: the thread's sum fits 64 bits
  if (row_top + (1 << 26) < NR) {  // uniform: -inf's bin (t = -2^30) lies inside the window
#pragma unroll
    for (int k = 0; k < EPT; k++) w[k] = kept_weight<true>(xv[k], tv[k], te[k], row_top, cR, cC, (uint32_t)(lo + t0 + k));
  } else {
#pragma unroll
    for (int k = 0; k < EPT; k++) w[k] = kept_weight<false>(xv[k], tv[k], te[k], row_top, cR, cC, (uint32_t)(lo + t0 + k));
  }
#pragma unroll
  for (int k = 0; k < EPT; k++) loc += w[k];
  u128 tot;
  const u128 incl = block_scan_incl_u128<NWV2>((u128)loc, L.red, &tot);
  const u128 c0 = incl - loc;
  if (c0 <= tl && tl < incl) {
    const uint64_t t = (uint64_t)(tl - c0);  // < loc
    uint64_t run = 0;
#pragma unroll
    for (int k = 0; k < EPT; k++) {
      if (w[k] && run <= t && t < run + w[k]) st.si[2] = lo + t0 + k;
      run += w[k];
    }
  }
  bar();
  return st.si[2];
}

// The step of a row that drew `tok`, on the device (qws_batch.advance): the token added to the row's state slot as
// qws_state_note adds one token (its block's entry counted, saturating, or appended), then the row's ngen and
// position incremented in the row array.  When tok lies in block g_pre, n_pre / e_pre are that block's entry count
// and this thread's first entry (entry threadIdx.x), loaded ahead.  All threads (tok and the row uniform); ends with
// the row written.
__device__ __forceinline__ void advance_row(const qws_batch& B, const qws_row& R, int row, int tok, int* s_hit, int g_pre, int n_pre, uint32_t e_pre) {
  if (tok < 0) return;
  const int slot = row_state(B, R);
  if (slot >= 0) {
    const int g = tok / BLK;
    const uint32_t local = (uint32_t)(tok - g * BLK);
    uint32_t* cnt = state_counts(B.state_mem, B.V, slot);
    uint32_t* ent = state_entries(B.state_mem, B.V, slot, g);
    const bool pre = g == g_pre;
    const int n0 = min(pre ? n_pre : (int)cnt[g], BLK);
    if (threadIdx.x == 0) *s_hit = -1;
    bar();
    for (int j = (int)threadIdx.x; j < n0; j += NT2)
      if (((pre && j < NT2 ? e_pre : ent[j]) & SE_LOCAL) == local) *s_hit = j;  // distinct tokens: one writer at most
    bar();
    if (threadIdx.x == 0) {
      const int j = *s_hit;
      if (j >= 0) {
        const uint32_t e = ent[j];
        ent[j] = (e & ((1u << SE_CNT_SHIFT) - 1u)) | (min((e >> SE_CNT_SHIFT) + 1u, SE_CNT_MAX) << SE_CNT_SHIFT);
      } else {
        const uint32_t p = atomicAdd(&cnt[g], 1u);
        if (p < (uint32_t)BLK) ent[p] = local | (1u << SE_CNT_SHIFT);
      }
    }
  }
  if (threadIdx.x == 0) {
    qws_row* rw = const_cast<qws_row*>(B.rows) + row;
    rw->ngen = R.ngen + 1;
    rw->position = R.position + 1u;
  }
}

// VER: the rows of a verify call (rres != nullptr)
template <int DT, bool VER>
__global__ void __launch_bounds__(NT2) k_resolve(qws_batch B, int G, char* ws, RowRes* rres) {
  __shared__ __attribute__((aligned(16))) unsigned long long s_fb[MAXG * FB];
  __shared__ unsigned long long s_emu[MAXG * NEXP];
  __shared__ uint64_t s_ec[XG];
  __shared__ uint32_t s_em[XG];
  __shared__ __attribute__((aligned(16))) uint32_t s_big[BIGW];
  __shared__ int s_nt;
  __shared__ __attribute__((aligned(16))) float2 s_ts[1024];
  __shared__ BI s_bi[MAXG];
  __shared__ RS s_st;
  __shared__ u128 s_red[NWV2 + 1];
  RL L;
  L.bi = s_bi;
  L.st = &s_st;
  L.ts = s_ts;
  L.big = s_big;
  L.fb = s_fb;
  L.emu = s_emu;
  L.ec = s_ec;
  L.em = s_em;
  L.nt = &s_nt;
  L.red = s_red;
  __shared__ qws_batch s_B;  // LDS copies the non-inlined block stager reads
  __shared__ qws_row s_R;
  RS& st = s_st;
  // Workgroup i runs on XCD i % 8 (round-robin dispatch): it takes a row whose blocks k_scan ran on that XCD (rows
  // [x * RB, (x + 1) * RB) there, RB = ceil(B / 8)), so the row's records are read back through the L2 that wrote them.
  const int RB = (B.B + NXCD - 1) / NXCD;
  const int row = (int)(blockIdx.x % NXCD) * RB + (int)(blockIdx.x / NXCD), tid = threadIdx.x;
  if (row >= B.B) return;  // whole workgroups, before any barrier
  // ---- round 1: every block header and the exp2 table into LDS (the headers in the fine-bin region).  All loads,
  // the row's parameters included, are issued before any is waited for.
  constexpr int HW = (int)(HDR_BYTES / 16), HPT = MAXG * HW / NT2;  // header words per thread
  static_assert(MAXG * HW % NT2 == 0 && 512 <= NT2, "round 1 layout");
  vu4 hv[HPT];
#pragma unroll
  for (int k = 0; k < HPT; k++) {
    const int i = tid + k * NT2;
    if (i < G * HW) hv[k] = gmem((const vu4*)rec_of(ws, G, row, i / HW))[i % HW];
  }
  vu4 tv;
  if (tid < 512) tv = gmem((const vu4*)EXP2_TS)[tid];
  const qws_row R = B.rows[row];
  if (tid == 0) {
    s_B = B;
    s_R = R;
  }
  const qws_batch& BB = s_B;
  const qws_row& RR = s_R;
  const uint32_t u_draw = draw_u24(R.seed, R.position, R.stream, R.row_key, R.draw_word);  // the draw's Philox word
  if (tid < 512) ((vu4*)s_ts)[tid] = tv;
#pragma unroll
  for (int k = 0; k < HPT; k++) {
    const int i = tid + k * NT2;
    if (i < G * HW) ((vu4*)s_fb)[i] = hv[k];
  }
  if (tid < NEXP) {
    st.Rc[tid] = 0u;
    st.Rm[tid] = 0ull;
  }
  for (int i = tid; i < NBK; i += NT2) {
    st.fbc[i] = 0u;
    st.fbs[i] = 0ull;
  }
  if (tid == 0) {
    st.G = G;
    st.fpow = -1;
    st.gbin = -1;
    st.rescans = 0;
    st.fxn = 0;
  }
  bar();
  auto hdr = [&](int g) -> const Rec& { return *(const Rec*)((const char*)s_fb + (size_t)g * HDR_BYTES); };
  if (tid < 64) {  // the row's best: one wave max over the blocks (G <= 64: lane g reads block g)
    uint64_t v = 0;
    if (tid < G) {
      const Rec& H = hdr(tid);
      BI b;
      b.max_key = H.max_key;
      b.max_idx = H.max_idx;
      b.c = H.c;
      b.flags = H.flags;
      b.nbw = H.nbw;
      b.n_patch = (H.flags & RF_CAND) ? H.n_patch : -1;
      b.dn = -1;
      b.gcnt = b.goff = b.gsrc = b.gofs = 0;
      b.w0 = H.w0;
      b.w1 = H.w1;
      b.wa = H.wa;
      b.ea = H.ea;
      b.n_list = H.n_list;
      b.wcnt = 0;
      s_bi[tid] = b;
      if (H.flags & RF_CAND) v = comp(H.max_key, H.max_idx);
    }
    const uint64_t m = wave_max_u64(v);
    if (tid == 0) st.best = m;
  }
  bar();
  const uint64_t best = st.best;
  const float K = kscale(R.temperature);
  if (best == 0 || !(R.temperature > 0.0f) || !(K < INFINITY)) {  // no candidate, or a greedy row
    if (tid == 0) {
      B.out_tokens[row] = best == 0 ? 0 : (int)comp_idx(best);
      if (B.out_probs && best != 0) B.out_probs[(size_t)row * B.V + comp_idx(best)] = 1.0f;  // the point mass
      if (B.out_info) B.out_info[row] = 2;
      if (VER) {
        RowRes o = {};
        o.kind = best == 0 ? RR_EMPTY : RR_GREEDY;
        o.tok = B.out_tokens[row];
        rres[row] = o;
      }
    }
    // a row without a candidate emits token 0 (its greedy token) and takes the step with it, as qws_finish_rows does
    if (!VER && B.advance) advance_row(B, R, row, best == 0 ? 0 : (int)comp_idx(best), &s_nt, -1, 0, 0u);
    return;
  }
  const float tmax = tval(okey_val(comp_key(best)), K);
  const int N = tfloor(tmax) >> 10;
  const int row_top = N * FB + (FB - 1);
  if (tid == 0) {
    st.K = K;
    st.N = N;
    st.row_top = row_top;
  }
  // ---- the row's per-power sums: block power e is row power e + (N - c) (consecutive threads read consecutive powers
  // of one staged header: no bank conflicts; the sums by LDS atomics)
  for (int i = tid; i < G * NEXP; i += NT2) {
    const int g = i / NEXP, e = i - g * NEXP;
    const Rec& H = hdr(g);
    const bool samp = (H.flags & RF_SAMP) && N - H.c <= D_EXP;
    const unsigned long long mu = samp ? H.emu[e] : 0ull;
    s_emu[i] = mu;
    if (e == 0) s_bi[g].dn = samp ? N - H.c : -1;
    const int er = e + N - H.c;
    if (samp && er <= D_EXP && H.ecnt[e]) {
      atomicAdd(&st.Rc[er], H.ecnt[e]);
      atomicAdd(&st.Rm[er], mu);
      atomicAdd(&s_bi[g].wcnt, (int)H.ecnt[e]);
    }
  }
  bar();
  // ---- the cuts: min-p, then top-k, then top-p; kept = row bin r < cR, or r == cR and comp >= cC (cR = NR: none)
  int cR = NR;
  uint64_t cC = 0;
  u128 mb = 0;                    // mass (row units) of the bins above the cut
  unsigned long long kept_n = 0;  // candidates kept so far
  before_bin(L, NR, &mb, &kept_n);
  // candidates below the row's window (weight 0) still count for top-k: the window's count is a lower bound, and a
  // K at or beyond it keeps every weighted candidate
  auto bin_kept = [&](uint64_t cmin, bool by_mass) -> unsigned long long {  // kept count / mantissa sum of the gathered bin
    unsigned long long v = 0;
    for_bin<DT>(L, BB, RR, ws, row, [&](uint64_t c, uint32_t mu) {
      if (c >= cmin) v += by_mass ? (unsigned long long)mu : 1ull;
    });
    block_add_u64(st, v);
    return st.su[7];
  };
  if (R.min_p > 0.0f) {
    const float tcut = (float)((double)(tmax / 1024.0f) + R.log2_min_p) * 1024.0f;
    const int rc = row_top - (tfloor(tcut) >> 4);
    if (rc < NR) {
      stage_power(L, ws, row, rc >> 6);
      gather<DT, VER>(L, BB, RR, ws, row, rc);
      // kept: t >= tcut, a prefix of the bin in comp order
      unsigned long long v = 0;
      for_bin<DT>(L, BB, RR, ws, row, [&](uint64_t c, uint32_t) { v += tval(okey_val(comp_key(c)), K) >= tcut ? 1ull : 0ull; });
      block_add_u64(st, v);
      const unsigned long long nk = st.su[7];
      cR = rc;
      float xc;
      if (nk == 0) {
        cC = ~0ull;
      } else if (nk == (unsigned long long)st.gn) {
        cC = 0;
      } else if (first_x_t(tcut, K, &xc)) {  // the kept prefix from the threshold's value: no selection
        cC = (uint64_t)okey(xc) << 32;
      } else {
        select_in_bin<DT>(L, BB, RR, ws, row, false, nk);
        cC = st.su[4];
      }
      before_bin(L, rc, &mb, &kept_n);
      kept_n += nk;
    }
  }
  // With top-k beside min-p a block writes its bins only down to the shallower of its own min-p cut and its own K-th
  // candidate, so the count above the row's min-p cut is exact when it is below K and at least K otherwise: the cut
  // runs when K <= kept_n (at kept_n == K it keeps the same set)
  if (R.top_k > 0 && (unsigned long long)R.top_k <= kept_n) {
    int pk;
    unsigned long long before_p;
    pow_cross_cnt(L, (unsigned long long)R.top_k, &pk, &before_p);
    stage_power(L, ws, row, pk);
    u128 before_f;
    const int bk = pk * FB + fine_cross(L, false, (u128)before_p, (u128)(unsigned long long)R.top_k, &before_f);
    const unsigned long long need = (unsigned long long)R.top_k - (unsigned long long)before_f;
    cR = bk;
    uint64_t pref_unused;
    if (st.fcnt[bk & 63] == need) {  // the whole bin is kept (cC = 0): no gather
      cC = 0;
    } else if (!select_listed<DT>(L, BB, RR, ws, row, bk, false, need, &cC, &pref_unused)) {
      gather<DT, VER>(L, BB, RR, ws, row, bk);
      select_in_bin<DT>(L, BB, RR, ws, row, false, need);
      cC = st.su[4];
    }
  }
  // ---- a cut set (min-p / top-k) of at most 64 candidates, all in their blocks' lists (each block's bins from its top
  // down to the cut listed without a gap): wave 0 holds them, one per lane, and finishes the row -- the top-p cut over
  // their exact weights in value order, then the draw in index order -- with no other power staged, no kept masses
  // per block and no block of the draw.  The same definition as the path below; test flags that ask for rescans or
  // staged draws keep that path.
  const unsigned long long n_cut = (R.top_k > 0 && (unsigned long long)R.top_k <= kept_n) ? (unsigned long long)R.top_k : kept_n;
  __shared__ int s_fast, s_ftok, s_fcR;
  __shared__ unsigned long long s_fS[2], s_fcC;
  u128 S2;
  int tok = -1;
  bool fast = false;
  if (cR < NR && n_cut > 0 && n_cut <= 64 && st.fpow == (cR >> 6) &&
      !(R.test_flags & (QWS_TF_RESCAN | QWS_TF_STAGED_DRAW | QWS_TF_SPLIT_SELECT))) {  // uniform
    if (wave_id() == 0) {
      const int lane = lane_id();
      // lane g: the number of block g's list entries in its bins down to the cut's (bins 0 .. cb listed, no gap)
      int cnt = 0;
      bool ok = true;
      if (lane < G && s_bi[lane].dn >= 0) {
        const BI& b = s_bi[lane];
        const int cb = cR - FB * b.dn;  // the cut's bin among the block's own
        if (cb >= 0) {
          const unsigned long long wd = s_fb[lane * FB + (cR & 63)];
          ok = cb < b.nbw && b.w0 == 0 && cb <= b.w1 && (cb <= b.wa || b.ea == b.wa + 1) && bw_listed(wd);
          cnt = ok ? (int)(bw_off(wd) + bw_cnt(wd)) : 0;
        }
      }
      const int inc = wave_scan_incl<int>(cnt), tot = readlane<int>(inc, 63), exc = inc - cnt;
      int res = 0;
      if (__ballot(!ok) == 0ull && tot <= 64) {  // uniform in the wave
        // list entry `lane` of the concatenation: its block by a binary search over the inclusive counts (all lanes)
        int g = 0;
        for (int sft = 32; sft > 0; sft >>= 1) g += __shfl(inc, g + sft - 1) <= lane ? sft : 0;
        const int e0 = __shfl(exc, min(g, 63));
        uint64_t c = 0, w = 0;
        uint32_t idx = 0xFFFFFFFFu;
        int r = NR;
        if (lane < tot) {
          c = els_of(ws, G, row, g)[lane - e0];
          const float t = tval(okey_val(comp_key(c)), K);
          r = row_top - (tfloor(t) >> 4);
          if (r < cR || (r == cR && c >= cC)) w = rw1(weigh(t, L.ts).mu, r);
          idx = comp_idx(c);
        }
        if ((unsigned long long)__popcll(__ballot(w != 0)) == n_cut) {  // every kept candidate is here
          const u128 S = wave_sum_u128((u128)w);
          u128 s2 = S;
          uint64_t cK = cC;
          int rK = cR;
          uint64_t wk = w;  // the kept weight after top-p
          if (R.top_p < 1.0f) {
            const uint64_t TP = (uint64_t)floor((double)R.top_p * 4294967296.0);
            const u128 thr = mul_shr_ceil(S, TP, 32);
            if (thr > 0) {
              u128 above = 0;  // kept weight of the larger comps
              for (int j = 0; j < tot; j++) {  // uniform
                const uint64_t cj = readlane<uint64_t>(c, j), wj = readlane<uint64_t>(w, j);
                above += cj > c ? (u128)wj : (u128)0;
              }
              const int k = min(first_lane(w != 0 && above < thr && thr <= above + w), 63);  // thr <= S: one lane crosses
              cK = readlane<uint64_t>(c, k);
              rK = readlane<int>(r, k);
              s2 = readlane<u128>(above + w, k);
              wk = c >= cK ? w : 0;
            }
          }
          const u128 tt = mul_shr_floor(s2, u_draw, 24);
          u128 below = 0;  // kept weight of the lower indices
          for (int j = 0; j < tot; j++) {  // uniform
            const uint32_t ij = readlane<uint32_t>(idx, j);
            const uint64_t wj = readlane<uint64_t>(wk, j);
            below += ij < idx ? (u128)wj : (u128)0;
          }
          const int l = first_lane(wk != 0 && below <= tt && tt < below + wk);
          if (lane == 0) {
            s_ftok = l < 64 ? (int)readlane<uint32_t>(idx, l) : -1;
            s_fcR = rK;
            s_fcC = cK;
            s_fS[0] = (unsigned long long)s2;
            s_fS[1] = (unsigned long long)(s2 >> 64);
          }
          res = 1;
        }
      }
      if (lane == 0) s_fast = res;
    }
    bar();
    fast = s_fast != 0;
    if (fast) {
      tok = s_ftok;
      cR = s_fcR;
      cC = s_fcC;
      S2 = ld128(s_fS[0], s_fS[1]);
    }
  }
  int a_g = -1, a_n = 0;  // advance: the drawn block and its state entries, loaded before the draw
  uint32_t a_e = 0u;
  if (!fast) {
    bool kept_done = false;  // the kept mass of every block computed with the cut (topp_cut_fast)
    // cC = 0: every element of bin cR is kept, and the bin's words give its mass (the staged power is cR's)
    u128 S = mb;
    if (cR < NR) {
      unsigned long long cnt_unused;
      before_bin(L, cR, &mb, &cnt_unused);
      S = mb + shl128(cC == 0 ? st.fmu[cR & 63] : bin_kept(cC, true), D_EXP - (cR >> 6));
    }
    if (R.top_p < 1.0f) {
      const uint64_t TP = (uint64_t)floor((double)R.top_p * 4294967296.0);
      const u128 thr = mul_shr_ceil(S, TP, 32);
      if (thr > 0) {
        int pp;
        u128 before_p, before_f;
        pow_cross_mass(L, thr, &pp, &before_p);
        stage_power(L, ws, row, pp);
        const int bp = pp * FB + fine_cross(L, true, before_p, thr, &before_f);
        const int sh = D_EXP - pp;
        cR = bp;
        mb = before_f;
        if (st.fcnt[bp & 63] == 1) {  // the crossing bin holds one element: the cut, the whole bin kept (no gather)
          cC = 0;
          S = mb + ((u128)st.fmu[bp & 63] << sh);
        } else {
          // the crossing in mantissa units of the bin's power: sum of mu * 2^sh >= thr - before  <=>  sum of mu >= ceil(...)
          const u128 need = thr - before_f;
          const uint64_t tmu = (uint64_t)((need + (((u128)1 << sh) - 1)) >> sh);
          uint64_t pref;  // the selection's inclusive mantissa sum at the cut
          if (topp_cut_fast(L, RR, ws, row, bp, tmu, &cC, &pref)) {
            kept_done = true;
          } else if (!select_listed<DT>(L, BB, RR, ws, row, bp, true, tmu, &cC, &pref)) {
            gather<DT, VER>(L, BB, RR, ws, row, bp);
            select_in_bin<DT>(L, BB, RR, ws, row, true, tmu);
            cC = st.su[4];
            pref = st.su[5];
          }
          S = mb + ((u128)pref << sh);
        }
      }
    }
    S2 = S;
    // a verify row ends at S2: the verify kernels draw from p for the one row of a sequence that needs it
    if constexpr (!VER) {
      // ---- kept mass per block: its powers above the cut's, its fine bins above the cut's bin and its kept elements there
      // (sixteen threads per block; topp_cut_fast has computed them already)
      for (int g0 = 0; g0 < (kept_done ? 0 : G); g0 += NT2 / 16) {  // uniform
        const int g = g0 + (tid >> 4), j = tid & 15;
        u128 k = 0;
        if (g < G && s_bi[g].dn >= 0) {
          const BI& b = s_bi[g];
          const int pc = cR < NR ? (cR >> 6) : NEXP;
          for (int er = b.dn + j; er < pc; er += 16) k += shl128(s_emu[g * NEXP + er - b.dn], D_EXP - er);
          if (cR < NR) {
            const int sh = D_EXP - pc;
            for (int f = j; f < (cR & 63) + (cC == 0 ? 1 : 0); f += 16) k += shl128(bw_mu(s_fb[g * FB + f]), sh);
            if (cC != 0 && st.gstaged) {  // a partial cut: the gathered bin is cR's
              for (int i = b.gofs + j; i < b.gofs + (b.gsrc ? b.gcnt : 0); i += 16)
                if (s_ec[i] >= cC) k += (u128)s_em[i] << sh;
            }
          }
        }
        k = row16_scan_incl<u128>(k);  // a block's sixteen threads are one DPP row: its last lane holds the total
        if (g < G && j == 15) {
          st.Klo[g] = (unsigned long long)k;
          st.Khi[g] = (unsigned long long)(k >> 64);
        }
      }
      if (!kept_done) bar();
      if (!kept_done && cR < NR && cC != 0 && !st.gstaged) {  // a bin too large for LDS: its kept elements by block from the sources
        const int sh = D_EXP - (cR >> 6);
        for_bin<DT>(L, BB, RR, ws, row, [&](uint64_t c, uint32_t mu) {
          if (c >= cC) {
            const int g = (int)(comp_idx(c) / BLK);
            atomic_add_u128(&st.Klo[g], &st.Khi[g], (u128)mu << sh);
          }
        });
      }
      // ---- the draw: the block by its kept mass (index order), then the token inside it
      const u128 tt = mul_shr_floor(S2, u_draw, 24);
      int gs;   // every wave picks it from the final kept masses (no barrier)
      u128 tl;  // the target inside that block
      {
        const int lane = lane_id();
        const u128 k = lane < G ? ld128(st.Klo[lane], st.Khi[lane]) : (u128)0;
        const u128 incl = wave_scan_incl_u128(k);
        const int l = first_lane(k != 0 && tt < incl);
        gs = l < 64 ? l : -1;
        tl = l < 64 ? tt - readlane<u128>(incl - k, l) : (u128)0;
      }
      // advance: the drawn block's state entries loaded now, so that noting the token waits for nothing after the draw
      const int aslot = (!VER && B.advance) ? row_state(B, R) : -1;
      if (aslot >= 0 && gs >= 0) {  // uniform; entry tid lies inside the block's BLK entry words
        a_g = gs;
        a_n = (int)gmem(state_counts(B.state_mem, B.V, aslot))[gs];  // global loads: no LDS wait of the draw waits for them
        a_e = gmem(state_entries(B.state_mem, B.V, aslot, gs))[tid];
      }
      // the drawn block's kept set whole in its list (its bins listed from the top without a gap down to the cut's, at most
      // a wave of elements there): drawn from those by wave 0; else the block is staged and weighed
      int nlist = 65;
      if (gs >= 0 && s_bi[gs].w0 == 0 && !(R.test_flags & QWS_TF_STAGED_DRAW)) {  // uniform
        const BI& b = s_bi[gs];
        if (cR == NR) {
          // no cut: the block's candidates inside the weight window, a top-down prefix of its bins as the (gap-free) list
          // is, lie whole in the list iff they are no more than the list holds
          if ((b.wa >= b.w1 || b.ea == b.wa + 1) && b.wcnt <= b.n_list) nlist = b.n_list;
        } else if (st.fpow == (cR >> 6)) {  // the cut's power is the staged one
          const int cb = cR - FB * b.dn;    // the cut's bin among the block's own
          if (cb >= 0 && cb <= b.w1 && (cb <= b.wa || b.ea == b.wa + 1)) {  // bins 0 .. cb all listed
            const unsigned long long wd = s_fb[gs * FB + (cR & 63)];
            if (bw_listed(wd)) nlist = (int)(bw_off(wd) + bw_cnt(wd));
          }
        }
      }
      if (nlist <= 64) {
        if (wave_id() == 0) tok = draw_listed(L, ws, row, gs, nlist, cR, cC, tl);
      } else if (gs >= 0) {
        tok = draw_in_block<DT>(L, BB, RR, ws, row, gs, cR, cC, tl);
      }
    }
  }
  if (B.out_probs) {  // dense probabilities of the kept set (test-hook path), by rescans of every block
    using BL = Blk<DT, NT2>;
    const double S2d = (double)(uint64_t)(S2 >> 64) * 18446744073709551616.0 + (double)(uint64_t)S2;
    for (int g = 0; g < G; g++) {
      if (s_bi[g].dn < 0) continue;
      stage_block<DT>(L, BB, RR, ws, row, g);
      const float* xs = (const float*)s_big;
      const int t0 = tid * BL::EPT;
#pragma unroll
      for (int k = 0; k < BL::EPT; k++) {
        const float v = xs[big_at(t0) + k];
        if (v == -INFINITY) continue;
        const W w = weigh(tval(v, K), s_ts);
        const int r = row_top - w.bin();
        const uint32_t idx = (uint32_t)(g * BLK + t0 + k);
        if (r < NR && (r < cR || (r == cR && comp(okey(v), idx) >= cC))) B.out_probs[(size_t)row * B.V + idx] = (float)((double)rw1(w.mu, r) / S2d);
      }
      bar();
    }
  }
  if (tid == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = tok < 0 && (fast || !VER) ? -1 : (st.rescans ? 1 : 0);
    if (VER) {
      RowRes o;
      o.s_lo = (unsigned long long)S2;
      o.s_hi = (unsigned long long)(S2 >> 64);
      o.cC = cC;
      o.cR = cR;
      o.row_top = row_top;
      o.K = K;
      o.kind = tok < 0 && fast ? RR_FAIL : RR_SAMPLED;  // outside the one-wave finish tok = -1: not drawn here
      o.tok = tok;
      o.pad = 0;
      rres[row] = o;
    }
  }
  if (!VER && B.advance) {  // uniform
    __shared__ int s_tok;
    if (tid == 0) s_tok = tok;  // thread 0 holds the row's token (a listed draw leaves it in wave 0 only)
    bar();
    advance_row(B, R, row, s_tok, &s_nt, a_g, a_n, a_e);
  }
}

}  // namespace qws
