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

#include <atomic>
#include <mutex>

#include "qws_rows.h"

namespace qws {

constexpr int NT1S = 512, NT1L = 1024;        // k_scan workgroups: 3 per CU; one per CU when the grid fits one round
constexpr int NT2 = 512, NWV2 = NT2 / 64;    // k_resolve workgroup
constexpr int CAP = 1024;                    // elements a block may list
constexpr int MARGIN = 6;                    // top-p: fine bins listed on either side of the block's own boundary
constexpr int CTOP = 256;                    // elements of a block's top bins listed beside a window further down
constexpr int MAXG = 64;                     // blocks per row (V <= 524,288)
constexpr int NR = NBIN;                     // row bins with a nonzero weight (row-relative, 0 = the top)
constexpr int XN = 4096;                     // elements of one bin k_resolve holds in LDS
constexpr unsigned long long M40 = (1ull << 40) - 1;

// ---------------------------------------------------------------------------------------------- block record
enum : int { RF_CAND = 1, RF_SAMP = 2, RF_WIN = 4, RF_OVER = 8 };
// Bins of a block are top-down: rel = (c * 64 + 63) - fine bin, so rel 0..63 is the power of two 2^c of the block's
// best and rel >> 6 = e counts powers of two below it.  Elements with rel >= NBIN weigh nothing in any row window.
struct Rec {
  uint32_t max_key, max_idx;     // best candidate (okey, lowest index); KEY_NEGINF: none
  int c, flags;                  // power of two of the best; RF_*
  int rel_max, rel_min;          // bins of the best and of the lowest candidate with rel < NBIN
  int w0, w1;                    // window, rel w0..w1 (w0 <= w1 with RF_WIN): a bin word for each non-empty bin
  int wa;                        // its elements are listed in bins w0..wa and ea..w1 (all of them when ea <= wa + 1)
  uint32_t n_win;                // listed elements
  uint32_t pcnt, n_tab;          // elements of power of two w0 >> 6 above w0; non-empty window bins
  unsigned long long pmu;        // summed mantissas of the pcnt elements
  int n_patch, ea;               // processed touched tokens listed (-1: more than TCAP, rebuild from the lists); ea
  // Horner prefixes over the powers of two e = rel >> 6 (e = 0: the best's): for k = 0..35, pc[k] = candidates with
  // e <= k and P[k] = sum over them of mu * 2^(k - e) (< 2^74).  A row whose best is dn powers of two above this
  // block's weighs the block at P[35 - dn] (its elements with e > 35 - dn weigh nothing in the row).
  uint32_t pc[NEXP];
  uint32_t pad3[4];
  unsigned long long plo[NEXP], phi[NEXP];
};
constexpr size_t HDR_FIX = 64;   // the fields before pc (staged by the resolver)
constexpr size_t HDR_BYTES = 1024;
static_assert(sizeof(Rec) <= HDR_BYTES && offsetof(Rec, pc) == HDR_FIX && sizeof(Rec) % 16 == 0, "record header");
// then n_tab bin words (the window's non-empty bins in rel order): {rel - w0 | listed << 12 | offset << 13, count,
// summed mantissas}, then n_win elements comp(key, index) of the listed bins, bucketed by bin in the same order
constexpr size_t TAB_OFF = HDR_BYTES;
constexpr size_t EL_OFF = TAB_OFF + (size_t)CAP * 16;
constexpr size_t PATCH_OFF = EL_OFF + (size_t)CAP * 8;     // then n_patch patches {local index, processed value}
constexpr size_t REC_BYTES = PATCH_OFF + (size_t)TCAP * 8;
__device__ inline char* rec_of(char* ws, int G, int row, int g) { return ws + ((size_t)row * G + g) * REC_BYTES; }

// cumulative bin word of k_scan: count (bits 50..63) | non-empty bins (bits 32..49) | approximate mass (fp32 bits)
__device__ inline uint32_t cw_cnt(unsigned long long w) { return (uint32_t)(w >> 50); }
__device__ inline uint32_t cw_nz(unsigned long long w) { return (uint32_t)(w >> 32) & 0x3FFFFu; }
__device__ inline float cw_mass(unsigned long long w) { return __uint_as_float((uint32_t)w); }

// ---------------------------------------------------------------------------------------------- k_scan
template <int DT, int NT1>
__global__ void __launch_bounds__(NT1) k_scan(qws_batch B, int G, char* ws, VerifyIO VIO) {
  constexpr int NWV1 = NT1 / 64;
  using BL = Blk<DT, NT1>;
  constexpr int EPT = BL::EPT;
  constexpr int PB = 8;                                       // bins per thread in the bin scan
  constexpr int NSCAN = NBIN / PB;                            // threads of the bin scan
  static_assert(NBIN % PB == 0 && FB % PB == 0 && NSCAN <= NT1, "bin scan layout");
  static_assert(2 * NBIN * 8 >= BLK * 4, "the histogram region holds the processor table");
  // region A: the processor table (BLK words), then the histogram [NBIN] and the cumulative words [NBIN]
  __shared__ __attribute__((aligned(16))) unsigned long long s_a[2 * NBIN + 64];  // + a dummy bin per lane
  __shared__ __attribute__((aligned(16))) float2 s_ts[1024];
  __shared__ uint32_t s_ecnt[NEXP];
  __shared__ unsigned long long s_emu[NEXP];
  __shared__ float s_redf[NWV1];
  __shared__ float s_scf[NWV1];
  __shared__ uint32_t s_scu[NWV1];
  __shared__ uint32_t s_imin;
  __shared__ int s_nt, s_relmin, s_x0, s_x1, s_xc, s_xt, s_nl;
  __shared__ int s_win[8];
  __shared__ unsigned long long s_pm;

  const int row = blockIdx.x / G, g = blockIdx.x - row * G;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  const qws_row R = B.rows[row];
  char* rec = rec_of(ws, G, row, g);
  Rec* H = (Rec*)rec;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();

  float x[EPT];
  // the processor table fills the start of region A; the touched tokens are listed in the rest, from a bitmap in the
  // exp2 table's space.  No final barrier: the barrier of the block maximum below comes before the histogram's
  // writes into region A and the table's copy into s_ts.
  constexpr int LCAP2 = (int)((sizeof(s_a) - BLK * 4) / 4);
  static_assert(LCAP2 >= TCAP, "every block with patches lists its touched tokens");
  static_assert(sizeof(s_ts) >= BLK / 8, "room for the bitmap");
  load_processed<DT, NT1, true>(B, R, row, lo, hi, (uint32_t*)s_a, x, (uint2*)(rec + PATCH_OFF), &s_nt, (uint32_t*)s_a + BLK, LCAP2, false,
                                (uint32_t*)s_ts);
  if (VIO.vx) {  // verify rows: the processed value of the draft token this row verifies
    const int t = row % (VIO.K + 1);
    if (t < VIO.K) {
      const int vt = VIO.dtok[(row / (VIO.K + 1)) * VIO.K + t];
      if (vt >= lo && vt < hi) {
#pragma unroll
        for (int e = 0; e < EPT; e++) {
          if (lo + BL::local(e) == vt) {
            VIO.vx[row] = x[e];
            const int j = VIO.inv[vt];
            const int b = row / (VIO.K + 1);
            if (VIO.nchain && t >= VIO.nchain[b])
              VIO.vq[row] = 1.0f;  // a delta proposal: q(d) = 1
            else
              VIO.vq[row] = (j >= 0 && j < VIO.Vd) ? VIO.dprob[((size_t)b * VIO.K + t) * VIO.Vd + j] : 0.0f;
          }
        }
      }
    }
  }
  // the processed touched tokens are recorded as patches for the resolver's rescan of the block of the draw
  const int n_patch = !(R.proc_on && row_touches(B, R)) ? 0 : (s_nt <= TCAP ? s_nt : -1);
  if (B.out_logits) {
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const int i = lo + BL::local(e);
      if (i < hi) B.out_logits[(size_t)row * B.V + i] = x[e] + 0.0f;  // -0 as +0 (the reference's zero bias)
    }
  }
  // ---- best candidate: the largest value, lowest index
  float mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < EPT; e++) mloc = fmaxf(mloc, x[e]);
  const float mw = wave_max_f(mloc);
  if (lane == 0) s_redf[wave] = mw;
  if (tid == 0) {
    s_imin = 0xFFFFFFFFu;
    s_relmin = 0;
    s_nl = 0;
    s_x0 = NBIN;
    s_x1 = NBIN;
    s_xc = NBIN;
    s_xt = NBIN;
  }
  bar();
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
  bar();
  const uint32_t imax = s_imin;
  if (M == -INFINITY || !samp) {
    if (tid == 0) {
      H->max_key = M == -INFINITY ? KEY_NEGINF : okey(M);
      H->max_idx = M == -INFINITY ? 0u : imax;
      H->flags = M == -INFINITY ? 0 : RF_CAND;
      H->wa = -1;
      H->ea = 0;
      H->n_win = 0;
      H->n_tab = 0;
      H->n_patch = n_patch;
    }
    return;
  }
  // ---- exact histogram of the weights by fine bin, top-down from the best's power of two
  for (int i = tid; i < 512; i += NT1) ((uint4*)s_ts)[i] = ((const uint4*)EXP2_TS)[i];
  const int qm = tfloor(tval(M, K));
  const int c = qm >> 10;
  const int btop = c * FB + (FB - 1);
  const int r0 = btop - (qm >> 4);  // the best's bin: the first occupied one
  unsigned long long* hist = s_a;
  unsigned long long* cum = s_a + NBIN;
  for (int i = tid; i < NBIN; i += NT1) hist[i] = 0ull;
  if (tid < NEXP) {
    s_ecnt[tid] = 0u;
    s_emu[tid] = 0ull;
  }
  bar();
  uint32_t rp[EPT / 2];  // the elements' bins + 1 (16 bits each; 0: outside the weight window)
  uint32_t rlast1 = (uint32_t)r0 + 1;
  unsigned long long* hist1 = hist - 1;  // hist1[r + 1] = hist[r]
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    // -inf clamps to t = -2^30: far outside the window.  Branch-free: an element outside the window adds into its
    // lane's dummy bin (never read), so the table reads and the atomics of all elements pipeline.
    const W w = weigh(tval(x[e], K), s_ts);
    const int r1 = btop + 1 - w.bin();  // bin + 1 >= r0 + 1 >= 1
    const bool in = r1 <= NBIN;
    atomicAdd(&hist1[in ? r1 : 2 * NBIN + 1 + lane], (1ull << 40) | (unsigned long long)w.mu);
    const uint32_t rel1 = in ? (uint32_t)r1 : 0u;
    rlast1 = max(rlast1, rel1);
    if (e & 1)
      rp[e >> 1] |= rel1 << 16;
    else
      rp[e >> 1] = rel1;
  }
  const uint32_t rlast = wave_max_u32(rlast1) - 1u;
  if (lane == 0) atomicMax(&s_relmin, (int)rlast);
  bar();
  // ---- bin scan over the occupied bins [r0, r1]: each thread a contiguous run of bins.  Exact per-power-of-two
  // sums (one atomic per power of two a run touches), then cumulative count / non-empty bins / approximate mass.
  const int r1 = s_relmin;
  {
    const int pbd = (r1 - r0 + NT1) / NT1;
    const int b0 = r0 + tid * pbd, b1 = min(b0 + pbd, r1 + 1);
    uint32_t lc = 0, lz = 0;
    float lm = 0.0f;
    int ecur = b0 >> 6;
    uint32_t ec = 0;
    unsigned long long em = 0;
    for (int r = b0; r < b1; r++) {
      const unsigned long long h = hist[r];
      const uint32_t bc = (uint32_t)(h >> 40);
      const unsigned long long mu = h & M40;
      if ((r >> 6) != ecur) {
        if (ec) {
          atomicAdd(&s_ecnt[ecur], ec);
          atomicAdd(&s_emu[ecur], em);
        }
        ecur = r >> 6;
        ec = 0;
        em = 0;
      }
      ec += bc;
      em += mu;
      lc += bc;
      lz += bc ? 1u : 0u;
      lm += ldexpf((float)(uint32_t)(mu >> 14), 14 - (r >> 6));
    }
    if (ec) {
      atomicAdd(&s_ecnt[ecur], ec);
      atomicAdd(&s_emu[ecur], em);
    }
    // block scans of (count | non-empty << 16) and of the mass, sharing one barrier
    const uint32_t lcz = lc | (lz << 16);
    const uint32_t sc = wave_scan_incl<uint32_t>(lcz);
    const float sm = wave_scan_incl<float>(lm);
    if (lane == 63) {
      s_scu[wave] = sc;
      s_scf[wave] = sm;
    }
    bar();
    uint32_t cb = 0;
    float mb = 0.0f;
    for (int i = 0; i < wave; i++) {
      cb += s_scu[i];
      mb += s_scf[i];
    }
    const uint32_t cex = cb + sc - lcz;
    float rm = mb + sm - lm;
    uint32_t rc = cex & 0xFFFFu, rz = cex >> 16;
    for (int r = b0; r < b1; r++) {
      const unsigned long long h = hist[r];
      const uint32_t bc = (uint32_t)(h >> 40);
      rc += bc;
      rz += bc ? 1u : 0u;
      rm += ldexpf((float)(uint32_t)((h & M40) >> 14), 14 - (r >> 6));
      cum[r] = ((unsigned long long)rc << 50) | ((unsigned long long)rz << 32) | __float_as_uint(rm);
    }
  }
  bar();
  // cumulative words at any bin: none above r0, the block's totals below r1
  auto cnt_to = [&](int r) -> uint32_t { return r < r0 ? 0u : cw_cnt(cum[min(r, r1)]); };
  auto nz_to = [&](int r) -> uint32_t { return r < r0 ? 0u : cw_nz(cum[min(r, r1)]); };
  auto mass_to = [&](int r) -> float { return r < r0 ? 0.0f : cw_mass(cum[min(r, r1)]); };
  const bool topk = R.top_k > 0, topp = R.top_p < 1.0f, minp = R.min_p > 0.0f;
  // ---- the floor below which nothing of this block can be kept: the block's min_p cut (the row's cut is at or
  // above it) and its share of the row's top K (with room; the resolver verifies the guess)
  int floor_r = NBIN - 1;
  if (minp) {
    const float tcut = (float)((double)(tval(M, K) / 1024.0f) + R.log2_min_p) * 1024.0f;
    const int rm = btop - (((int)floorf(tcut)) >> 4);
    if (rm < NBIN) floor_r = max(rm, 0);
  }
  if (topk) {  // first bin whose cumulative count reaches kk
    const uint32_t kk = R.top_k <= 64 ? (uint32_t)R.top_k : (uint32_t)min(R.top_k, 2 * R.top_k / G + 64);
    for (int r = r0 + tid; r <= r1; r += NT1)
      if (cnt_to(r) >= kk && cnt_to(r - 1) < kk) s_x0 = r;
    bar();
    floor_r = min(floor_r, s_x0);
  }
  if (cnt_to(floor_r) > (uint32_t)CAP) {  // the first bin whose cumulative mass reaches top_p of the block's, and the
    // first bins whose cumulative counts exceed CAP and CTOP (listable top sets end before them)
    const float tgt = topp ? R.top_p * mass_to(floor_r) : 0.0f;
    for (int r = r0 + tid; r <= min(floor_r, r1); r += NT1) {
      if (topp && mass_to(r) >= tgt && mass_to(r - 1) < tgt) s_x1 = r;
      if (cnt_to(r) > (uint32_t)CAP && cnt_to(r - 1) <= (uint32_t)CAP) s_xc = r;
      if (cnt_to(r) > (uint32_t)CTOP && cnt_to(r - 1) <= (uint32_t)CTOP) s_xt = r;
    }
    bar();
  }
  // ---- thread 0: the window.  Its bin words cover bins w0..w1; its elements are listed in bins w0..wa and ea..w1.
  // A window around the block's own boundary also lists the elements of the block's top bins (up to CTOP of them,
  // bins up to wa) and gets words from the top (when they fit), so the row's boundary is pinned wherever it falls
  // between the block's top and its own boundary: near the top for a block far below the row's best, deeper for
  // the blocks that carry most of the row's mass.
  if (tid == 0) {
    int w0 = 0, w1 = -1, wa = -1, ea = 0, fl = 0;
    if (topk || topp || minp) {
      if (cnt_to(floor_r) <= (uint32_t)CAP) {
        w1 = floor_r;  // the whole top set
        wa = w1;
      } else {
        const int tp = min(s_xt - 1, floor_r);  // the top bins with at most CTOP elements
        const uint32_t budget = (uint32_t)CAP - (tp >= 0 ? cnt_to(tp) : 0u);
        int a = 0, bb = -1;
        if (topp) {
          const int rp_ = min(s_x1, floor_r);
          const int b = min(floor_r, rp_ + MARGIN);
          if (cnt_to(b) <= (uint32_t)CAP) {
            // the top set down to the block's own boundary fits: list it as deep as CAP allows
            w1 = max(b, min(floor_r, s_xc - 1));
            wa = w1;
          } else {
            a = max(0, rp_ - MARGIN);
            bb = b;
            while (a <= bb && cnt_to(bb) - cnt_to(a - 1) > budget) {
              if (bb - rp_ >= rp_ - a)
                bb--;
              else
                a++;
            }
          }
        } else {  // a min_p / top-k floor with more than CAP tokens above it: the bins just above the floor
          a = max(0, floor_r - 2 * MARGIN);
          bb = floor_r;
          while (a <= bb && cnt_to(bb) - cnt_to(a - 1) > budget) a++;
        }
        if (w1 < 0) {
          if (a <= bb) {
            // words from the top and the elements of the top bins when the top bins carry a real share of the block's
            // mass (a peaked block; in a flat row every block's boundary sits near the row's) and the words fit
            if (tp >= r0 && mass_to(tp) >= 0.25f * mass_to(floor_r) && nz_to(bb) - nz_to(r0 - 1) <= (uint32_t)CAP) {
              w0 = 0;
              w1 = bb;
              wa = tp;
              ea = a;
            } else {  // words and elements of [a, bb] only
              w0 = a;
              w1 = bb;
              wa = bb;
              ea = a;
            }
          } else {
            fl |= RF_OVER;
          }
        }
      }
    }
    const int eb = max(ea, wa + 1);  // first listed bin after the top part
    s_win[0] = w0;
    s_win[1] = w1;
    s_win[2] = fl | (w0 <= w1 ? RF_WIN : 0);
    s_win[3] = w0 <= w1 ? (int)(cnt_to(min(wa, w1)) - cnt_to(w0 - 1) + (eb <= w1 ? cnt_to(w1) - cnt_to(eb - 1) : 0u)) : 0;
    s_win[4] = w0 <= w1 ? (int)(nz_to(w1) - nz_to(w0 - 1)) : 0;
    s_win[5] = wa;
    s_win[6] = ea;
  }
  bar();
  const int w0 = s_win[0], w1 = s_win[1], fl = s_win[2], wa = s_win[5], ea = s_win[6];
  const int eb = max(ea, wa + 1);
  auto listed = [&](uint32_t rel) { return rel - (uint32_t)w0 <= (uint32_t)(w1 - w0) && ((int)rel <= wa || (int)rel >= eb); };  // rel < NBIN
  if (fl & RF_WIN) {
    const uint32_t z0 = nz_to(w0 - 1);
    // listed elements in bins w0 .. r - 1
    auto lbefore = [&](int r) -> uint32_t {
      return cnt_to(min(r - 1, wa)) - cnt_to(w0 - 1) + (r > eb ? cnt_to(r - 1) - cnt_to(eb - 1) : 0u);
    };
    // bin words of the window's non-empty bins (counts from the cumulative words, mantissas from the histogram's
    // low bits, which the placement below leaves unchanged).  A listed bin's histogram count becomes the end of its
    // elements in the record's list: the placement counts it down to each element's slot.
    uint4* TW = (uint4*)(rec + TAB_OFF);
    for (int r = w0 + tid; r <= w1; r += NT1) {
      const uint32_t cn = cnt_to(r) - cnt_to(r - 1);
      if (!cn) continue;
      const uint32_t slot = nz_to(r - 1) - z0;
      const unsigned long long mu = hist[r] & M40;
      const bool lr = listed((uint32_t)r);
      const uint32_t lb = lbefore(r);
      TW[slot] = make_uint4((uint32_t)(r - w0) | (lr ? 1u << 12 : 0u) | (lb << 13), cn, (uint32_t)mu, (uint32_t)(mu >> 32));
      if (lr) hist[r] = ((unsigned long long)(lb + cn) << 40) | mu;
    }
    // elements of the window, bucketed by bin: first compacted into LDS as {local index, value bits} (the exp2
    // table's space, CAP entries; one atomic per wave), then placed one per thread as comps: the k-th arrival in a
    // listed bin whose elements end at slot m takes slot m - k (the count field of the histogram word counts down)
    uint64_t* EL = (uint64_t*)(rec + EL_OFF);
    uint64_t* LW = (uint64_t*)s_ts;
    static_assert(CAP * 8 <= sizeof(s_ts), "window list in the table's space");
    auto wave_base = [&](int nw) {  // this lane's first slot in LW: one atomic per wave
      const int inc = wave_scan_incl<int>(nw);
      int wb = 0;
      if (lane == 63 && inc) wb = atomicAdd(&s_nl, inc);
      return readlane<int>(wb, 63) + inc - nw;
    };
    auto rel1_of = [&](int e) { return (rp[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu; };  // bin + 1, 0 outside
    if (eb == wa + 1 || wa >= w1) {
      // no unlisted bins inside the window: one range test per element (0 wraps past span), counted, then every
      // element written without a branch, the unlisted ones into the lane's dummy histogram bin (never read)
      const uint32_t span = (uint32_t)(w1 - w0), b1 = (uint32_t)(w0 + 1);
      int nw = 0;
#pragma unroll
      for (int e = 0; e < EPT; e++) nw += rel1_of(e) - b1 <= span ? 1 : 0;
      uint64_t* dst = LW + wave_base(nw);
      uint64_t* dummy = (uint64_t*)(s_a + 2 * NBIN + lane);
#pragma unroll
      for (int e = 0; e < EPT; e++) {
        const bool l = rel1_of(e) - b1 <= span;
        *(l ? dst : dummy) = ((uint64_t)__float_as_uint(x[e]) << 32) | (uint32_t)BL::local(e);
        dst += l ? 1 : 0;
      }
    } else {
      uint32_t lm = 0;  // bit e: element e is listed
#pragma unroll
      for (int e = 0; e < EPT; e++) lm |= listed(rel1_of(e) - 1u) ? 1u << e : 0u;  // 0 - 1: never listed
      int off = wave_base(__popc(lm));
#pragma unroll
      for (int e = 0; e < EPT; e++)
        if ((lm >> e) & 1u) LW[off++] = ((uint64_t)__float_as_uint(x[e]) << 32) | (uint32_t)BL::local(e);
    }
    bar();
    for (int i = tid; i < s_win[3]; i += NT1) {
      const uint64_t lw = LW[i];
      const float v = __uint_as_float((uint32_t)(lw >> 32));
      const int rel = btop - (tfloor(tval(v, K)) >> 4);
      const unsigned long long old = atomicAdd(&hist[rel], (unsigned long long)(-(1ll << 40)));
      EL[(uint32_t)(old >> 40) - 1] = comp(okey(v), (uint32_t)lo + (uint32_t)lw);
    }
    // elements of power of two w0 >> 6 above w0
    if (wave == 0 && (w0 & 63)) {
      const int u = w0 >> 6;
      const unsigned long long h = lane < (w0 & 63) ? hist[u * FB + lane] & M40 : 0ull;
      const unsigned long long pm = wave_sum<unsigned long long>(h);
      if (lane == 0) s_pm = pm;
    }
  }
  if (tid == 0 && !((fl & RF_WIN) && (w0 & 63))) s_pm = 0ull;
  bar();
  if (tid == 0) {
    H->max_key = okey(M);
    H->max_idx = imax;
    H->c = c;
    H->flags = RF_CAND | RF_SAMP | fl;
    H->rel_max = r0;
    H->rel_min = s_relmin;
    H->w0 = w0;
    H->w1 = w1;
    H->wa = s_win[5];
    H->ea = s_win[6];
    H->n_win = (uint32_t)s_win[3];
    H->n_tab = (uint32_t)s_win[4];
    H->pcnt = (fl & RF_WIN) && (w0 & 63) ? cnt_to(w0 - 1) - cnt_to((w0 & ~63) - 1) : 0u;
    H->pmu = s_pm;
    H->n_patch = n_patch;
  }
  if (tid < 64) {  // the Horner prefixes by one wave scan: S_k = sum_{e <= k} emu[e] * 2^(35 - e) = P[k] * 2^(35 - k)
    const u128 v = tid < NEXP ? shl128(s_emu[tid], D_EXP - tid) : (u128)0;
    const u128 S = wave_scan_incl_u128(v);
    const uint32_t n = wave_scan_incl<uint32_t>(tid < NEXP ? s_ecnt[tid] : 0u);
    const u128 P = shr128(S, D_EXP - min(tid, D_EXP));
    if (tid < NEXP) {
      H->pc[tid] = n;
      H->plo[tid] = (unsigned long long)P;
      H->phi[tid] = (unsigned long long)(P >> 64);
    }
  }
}

// ---------------------------------------------------------------------------------------------- k_resolve
// One workgroup per row.  Global loads are issued in few parallel rounds (headers, bin words, one bin's elements,
// the block of the draw); the per-block work then runs from LDS.
constexpr int WCAP = 2048;       // bin words staged in LDS
constexpr int NBK_LOG = 9;
constexpr int NBK = 1 << NBK_LOG; // comp buckets of a round of the in-bin selection
static_assert(MAXG * HDR_FIX <= BLK * 4 && WCAP * 16 <= BLK * 4, "staging region");
// whole headers are staged when G of them fit the staging region (G <= 40), else their fixed fields only

struct BH {                      // a block's record as the resolver uses it
  uint32_t max_key, max_idx;
  int c, flags, rel_max, rel_min, w0, w1;
  uint32_t n_win, n_tab;
  int wt;                        // rel of the first bin word (the window's w0 as k_scan chose it)
  int d;                         // row bin of the block's rel 0: (N - c) * 64
  int active;                    // some candidate of the block weighs in the row
  int listed;                    // its window is usable: row bins d + w0 .. d + w1 are listed completely
  int mode;                      // kept mass at the cut: 0 nothing, 1 above-window + window part, 2 all
  int woff;                      // first word of the block in the row's flat word order
  int n_patch;
  int eoff, ecnt;                // element range of the bin being gathered
  int rs;                        // the bin being gathered holds elements this block did not list: rescan it
  int ebase;                     // its offset in the gathered list
};

struct RS {                      // row state (LDS)
  int N, row_top, G, nw;
  float K, tmax;
  unsigned long long best;
  unsigned long long Tlo[MAXG], Thi[MAXG], Alo[MAXG], Ahi[MAXG], Klo[MAXG], Khi[MAXG];
  uint32_t nT[MAXG], nA[MAXG];
  int cR;                        // cut: kept = R < cR, or R == cR and comp >= cC (cR = NR: no cut)
  unsigned long long cC;
  int found;
  int wstaged;                   // the bin words are staged in L.big (a block rescan clears this)
  int wmore;                     // some listed block has more bin words than the first round loads
  unsigned long long t_lo, t_hi; // scratch u128
  unsigned long long u0, u1, kmin, kmax;
  int rhi;                       // the last row bin holding a candidate of an active block (first pass)
  int si[8];
  uint32_t bcnt[NBK];
  unsigned long long bsum[NBK];
};

struct KL {                      // k_resolve LDS views
  unsigned long long *mlo, *mhi; // [NR] row-bin masses (row units), then inclusive prefix
  uint32_t* cnt;                 // [NR] counts, then prefix
  int* good;                     // [NR + 1] difference array of blocks pinning a bin, then the count
  uint64_t* xs;                  // [64] the last elements of an in-bin selection: comp
  uint64_t* xv;                  // [64]                                            value
  uint64_t* ec;                  // [XN] elements of one bin: comp
  uint32_t* em;                  // [XN] their mantissas
  uint32_t* big;                 // [BLK] staged headers, then staged words, then a block (processor table / values)
  int* nt;
  float2* ts;
  BH* bh;
  RS* st;
  u128* red;
  uint32_t* redu;
  uint64_t* red64;
  int rhi;                       // the row bins hold [0, rhi]: every candidate of the row lies there, so the
                                 // prefixes past rhi equal rhi's and every block pins those bins
};

__device__ inline u128 ld128(unsigned long long lo, unsigned long long hi) { return ((u128)hi << 64) | lo; }
__device__ inline u128 Cm(const KL& L, int r) { return r < 0 ? (u128)0 : ld128(L.mlo[min(r, L.rhi)], L.mhi[min(r, L.rhi)]); }
__device__ inline uint32_t Cn(const KL& L, int r) { return r < 0 ? 0u : L.cnt[min(r, L.rhi)]; }
__device__ inline bool Good(const KL& L, int r) { return r >= 0 && r < NR && (r > L.rhi || L.good[r] == L.st->G); }
// row weight of a sum of mantissas in row bin r: mu * 2^(35 - (r >> 6))
__device__ inline u128 rw(uint64_t mu, int r) { return shl128(mu, D_EXP - (r >> 6)); }
// row weight of one mantissa (< 2^25, so the weight fits 64 bits: a 64-bit shift)
__device__ inline uint64_t rw1(uint32_t mu, int r) { return (uint64_t)mu << (D_EXP - (r >> 6)); }
__device__ inline void st128(unsigned long long* lo, unsigned long long* hi, u128 v) {
  *lo = (unsigned long long)v;
  *hi = (unsigned long long)(v >> 64);
}
__device__ inline const uint64_t* els_of(char* ws, int G, int row, int g) { return (const uint64_t*)(rec_of(ws, G, row, g) + EL_OFF); }
// bin word k of block g: staged (the row's words fit WCAP) or from the record
__device__ inline uint4 word_of(const KL& L, char* ws, int row, int g, uint32_t k) {
  const RS& st = *L.st;
  if (st.wstaged) return ((const uint4*)L.big)[L.bh[g].woff + k];
  return ((const uint4*)(rec_of(ws, st.G, row, g) + TAB_OFF))[k];
}
// block of flat word / element index i given per-block starts (ascending) in field F
template <typename F>
__device__ inline int block_at(const KL& L, int G, int i, F start) {
  int a = 0, b = G - 1;
  while (a < b) {
    const int m = (a + b + 1) >> 1;
    if (start(L.bh[m]) <= i)
      a = m;
    else
      b = m - 1;
  }
  return a;
}

// Calls fn(block, word) for every bin word of the listed blocks, flat over the row.  KW words per thread are loaded
// together (from global when the words are not staged), then processed.
template <typename F>
__device__ __forceinline__ void for_words(const KL& L, char* ws, int row, F fn) {
  constexpr int KW = 8;
  const RS& st = *L.st;
  const int G = st.G, nw = st.nw;
  for (int i0 = 0; i0 < nw; i0 += NT2 * KW) {
    uint4 wv[KW];
    int gk[KW];
#pragma unroll
    for (int k = 0; k < KW; k++) {
      const int i = i0 + (int)threadIdx.x + k * NT2;
      gk[k] = -1;
      if (i < nw) {
        const int g = block_at(L, G, i, [](const BH& h) { return h.woff; });
        gk[k] = g;
        wv[k] = word_of(L, ws, row, g, (uint32_t)(i - L.bh[g].woff));
      }
    }
#pragma unroll
    for (int k = 0; k < KW; k++)
      if (gk[k] >= 0) fn(gk[k], wv[k]);
  }
}

// first row bin whose inclusive prefix reaches target (mass or count): the unique r with C(r) >= t > C(r - 1)
template <bool MASS>
__device__ __forceinline__ int first_cross(const KL& L, u128 target) {
  if (threadIdx.x == 0) L.st->found = NR;
  bar();
  for (int r = threadIdx.x; r <= L.rhi; r += NT2) {  // past rhi the prefixes no longer grow
    const u128 v = MASS ? Cm(L, r) : (u128)Cn(L, r);
    const u128 p = MASS ? Cm(L, r - 1) : (u128)Cn(L, r - 1);
    if (v >= target && p < target) L.st->found = r;
  }
  bar();
  const int r = L.st->found;
  bar();
  return r;
}

// Wave 0: the bucket (0 = the largest comps) where base + the prefix of the bucket values crosses target: st.si[4]
// (-1: never), the value before it in st.u0 and its element count in st.si[5].  Ends with a barrier.
// The smallest sh with (range >> sh) < NBK: the bucket width of a round over a comp range
__device__ inline int bucket_shift(uint64_t range) {
  const int bits = range ? 64 - __clzll((long long)range) : 0;
  return max(bits - NBK_LOG, 0);
}

// Slot of this lane's item in a list appended to by the whole wave (all 64 lanes active): one atomic per wave
__device__ inline int wave_append(bool take, int* count) {
  const uint64_t m = __ballot(take);
  int b = 0;
  if (lane_id() == 0 && m) b = atomicAdd(count, __popcll(m));
  return readlane<int>(b, 0) + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Publishes a range holding every comp of a gathered list (st.kmin / st.kmax, cleared by the gather) from each
// thread's smallest and largest value key: comps key << 32 | any index part (u32 reductions are cheaper than u64 ones;
// the range is the exact one widened to whole keys)
__device__ inline void publish_range(RS& st, uint32_t kmin, uint32_t kmax) {
  kmin = ~wave_max_u32(~kmin);
  kmax = wave_max_u32(kmax);
  if (lane_id() == 0 && kmin <= kmax) {
    atomicMin(&st.kmin, (unsigned long long)kmin << 32);
    atomicMax(&st.kmax, ((unsigned long long)kmax << 32) | 0xFFFFFFFFull);
  }
}

// Clears the gather count, the rescan flag, the comp range and the buckets of the selection that follows a gather
// (before a barrier)
__device__ inline void clear_gather(RS& st) {
  if (threadIdx.x == 0) {
    st.si[0] = 0;
    st.si[3] = 0;
    st.kmin = ~0ull;
    st.kmax = 0;
  }
  for (int i = threadIdx.x; i < NBK; i += NT2) {
    st.bcnt[i] = 0;
    st.bsum[i] = 0;
  }
}

__device__ __forceinline__ void crossing_bucket(const KL& L, uint64_t base, uint64_t target) {
  RS& st = *L.st;
  if (wave_id() == 0) {
    const int lane = lane_id();
    uint64_t v[NBK / 64], loc = 0;
#pragma unroll
    for (int k = 0; k < NBK / 64; k++) {
      v[k] = st.bsum[lane * (NBK / 64) + k];
      loc += v[k];
    }
    const uint64_t incl = wave_scan_incl<uint64_t>(loc);
    uint64_t run = base + incl - loc;
    int hit = -1;
    uint64_t before = 0;
#pragma unroll
    for (int k = 0; k < NBK / 64; k++) {
      if (hit < 0 && run + v[k] >= target) {
        hit = lane * (NBK / 64) + k;
        before = run;
      }
      run += v[k];
    }
    const int l = first_lane(hit >= 0);
    if (lane == l) {
      st.si[4] = hit;
      st.u0 = before;
      st.si[5] = (int)st.bcnt[hit];
    }
    if (l == 64 && lane == 0) st.si[4] = -1;
  }
  bar();
}

// Weighted selection among the n gathered elements (ec / em, any order): in comp-descending order, the first
// element whose inclusive prefix of value (1 per element, or its mantissa) reaches target (>= 1).  Returns its comp
// and, in *incl, that inclusive prefix; ok = false when the target exceeds the total.  The gather leaves the
// buckets and the range cleared.  A radix refinement on the
// whole comp (value key, then index): each round buckets the elements of the current comp range by NBK equal
// ranges, finds the bucket where the prefix crosses the target and narrows the range to it, until one element is
// left.
struct Sel {
  uint64_t c;
  uint64_t incl;
  bool ok;
};
__device__ __forceinline__ Sel select_in_bin(const KL& L, int n, bool by_mass, uint64_t target) {
  RS& st = *L.st;
  const int tid = threadIdx.x;
  Sel out;
  out.ok = false;
  out.c = 0;
  out.incl = 0;
  if (n <= 64) {  // at most a wave of elements: wave 0 ranks them directly (each lane against all others)
    if (wave_id() == 0) {
      const int lane = lane_id();
      const uint64_t c = lane < n ? L.ec[lane] : 0ull;
      const uint64_t v = lane < n ? (by_mass ? (uint64_t)L.em[lane] : 1ull) : 0ull;
      uint64_t above = 0;  // value of the elements with a larger comp
      for (int j = 0; j < n; j++) {
        const uint64_t cj = readlane<uint64_t>(c, j), vj = readlane<uint64_t>(v, j);
        above += cj > c ? vj : 0ull;
      }
      const bool hit = lane < n && above < target && above + v >= target;
      const int l = first_lane(hit);
      if (lane == l) {
        st.u1 = c;
        st.t_lo = above + v;
      }
      if (lane == 0) st.si[6] = l < 64 ? 1 : 0;
    }
    bar();
    out.ok = st.si[6] != 0;
    out.c = st.u1;
    out.incl = st.t_lo;
    bar();
    return out;
  }
  {  // the first range: the elements' value keys' range
    uint32_t lmin = ~0u, lmax = 0;
    for (int i = tid; i < n; i += NT2) {
      const uint32_t k = comp_key(L.ec[i]);
      lmin = min(lmin, k);
      lmax = max(lmax, k);
    }
    publish_range(st, lmin, lmax);
  }
  bar();
  uint64_t kmin = st.kmin, kmax = st.kmax, base = 0;
  if (kmin > kmax) return out;  // no elements
  for (int round = 0; round < 16; round++) {
    const int sh = bucket_shift(kmax - kmin);
    for (int i = tid; i < n; i += NT2) {
      const uint64_t c = L.ec[i];
      if (c >= kmin && c <= kmax) {
        const int b = NBK - 1 - (int)((c - kmin) >> sh);  // bucket 0 = the largest comps
        atomicAdd(&st.bcnt[b], 1u);
        atomicAdd(&st.bsum[b], by_mass ? (unsigned long long)L.em[i] : 1ull);
      }
    }
    bar();
    crossing_bucket(L, base, target);
    const int hb = st.si[4];
    if (hb < 0) break;  // the target exceeds the total
    base = st.u0;
    const int nb = st.si[5];
    const uint64_t bl = kmin + ((uint64_t)(NBK - 1 - hb) << sh);
    const uint64_t span = (1ull << sh) - 1;  // sh < 64: range < 2^64
    const uint64_t bh = kmax - bl <= span ? kmax : bl + span;
    for (int i = tid; i < NBK; i += NT2) {
      st.bcnt[i] = 0;
      st.bsum[i] = 0;
    }
    if (nb <= 64) {  // at most a wave of elements left: wave 0 ranks them directly
      if (tid == 0) st.si[5] = 0;
      bar();
      for (int i = tid; i < n; i += NT2) {  // few of them: one atomic per element
        const uint64_t c = L.ec[i];
        if (c >= bl && c <= bh) {
          const int p = atomicAdd(&st.si[5], 1);
          L.xs[p] = c;
          L.xv[p] = by_mass ? (uint64_t)L.em[i] : 1ull;
        }
      }
      bar();
      if (wave_id() == 0) {
        const int lane = lane_id();
        const uint64_t c = lane < nb ? L.xs[lane] : 0ull;
        const uint64_t v = lane < nb ? L.xv[lane] : 0ull;
        uint64_t above = 0;  // value of the elements with a larger comp
        for (int j = 0; j < nb; j++) {
          const uint64_t cj = readlane<uint64_t>(c, j), vj = readlane<uint64_t>(v, j);
          above += cj > c ? vj : 0ull;
        }
        const bool hit = lane < nb && base + above < target && base + above + v >= target;
        const int l = first_lane(hit);
        if (lane == l) {
          st.u1 = c;
          st.t_lo = base + above + v;
        }
      }
      bar();
      out.ok = true;
      out.c = st.u1;
      out.incl = st.t_lo;
      bar();
      return out;
    }
    kmin = bl;
    kmax = bh;
    bar();
  }
  bar();
  return out;
}

// Block g of the row, processed, into x (Blk<DT, NT2> layout).  With the block's patches recorded by k_scan the raw
// logits get the mask and the patches (staged through L.big; the patches load together with the logits);
// otherwise the processors are rebuilt from the row's lists.  Ends with a barrier; L.big is free afterwards.
template <int DT>
__device__ __forceinline__ void load_block(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int g, float (&x)[Blk<DT, NT2>::EPT],
                                           bool staged = false) {
  using BL = Blk<DT, NT2>;
  const RS& st = *L.st;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  const int np = L.bh[g].n_patch;
  if (!R.proc_on || np < 0) {
    load_processed<DT, NT2>(B, R, row, lo, hi, L.big, x, nullptr, L.nt);
    bar();
    if (staged) {
      float* xs = (float*)L.big;
#pragma unroll
      for (int e = 0; e < BL::EPT; e++) xs[BL::local(e)] = x[e];
      bar();
    }
    return;
  }
  constexpr int PPT = TCAP / NT2;  // patches per thread
  uint2 pv[PPT];
  const uint2* PT = (const uint2*)(rec_of(ws, st.G, row, g) + PATCH_OFF);
#pragma unroll
  for (int k = 0; k < PPT; k++) {
    const int p = (int)threadIdx.x + k * NT2;
    pv[k] = p < np ? PT[p] : make_uint2(0xFFFFFFFFu, 0u);
  }
  BL::load(B, row, lo, hi, x);
  BL::mask(B, R, lo, hi, x);
  if (np > 0 || staged) {
    float* xs = (float*)L.big;
#pragma unroll
    for (int e = 0; e < BL::EPT; e++) xs[BL::local(e)] = x[e];
    if (np > 0) {
      bar();
#pragma unroll
      for (int k = 0; k < PPT; k++)
        if (pv[k].x != 0xFFFFFFFFu) xs[pv[k].x] = __uint_as_float(pv[k].y);
    }
    if (staged) {
      bar();
      return;
    }
    bar();
#pragma unroll
    for (int e = 0; e < BL::EPT; e++) x[e] = xs[BL::local(e)];
  }
  bar();
}

// Calls fn(block, cmp, row bin, mu) for every candidate of the row with a nonzero row weight, block by block, and
// end(block) after each block (all threads).
template <int DT, typename F, typename E>
__device__ __forceinline__ void for_rescan(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, F fn, E end) {
  using BL = Blk<DT, NT2>;
  const RS& st = *L.st;
  for (int g = 0; g < st.G; g++) {
    if (!L.bh[g].active) continue;
    const int lo = g * BLK;
    float x[BL::EPT];
    load_block<DT>(L, B, R, ws, row, g, x);
#pragma unroll
    for (int e = 0; e < BL::EPT; e++) {
      if (x[e] == -INFINITY) continue;
      const W w = weigh(tval(x[e], st.K), L.ts);
      const int r = st.row_top - w.bin();
      if (r < NR) fn(g, comp(okey(x[e]), (uint32_t)(lo + BL::local(e))), r, w.mu);
    }
    end(g);
    bar();
  }
}

// Weighted selection inside row bin r among its elements with comp >= cmin when the bin holds more than XN of them:
// radix rounds over rescans of the row (each counts the elements of the current comp range into NBK buckets) until
// the crossing bucket fits LDS, whose elements one more rescan gathers for select_in_bin.
template <int DT>
__device__ __forceinline__ Sel select_rescan(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int r, uint64_t cmin, bool by_mass,
                                          uint64_t target) {
  RS& st = *L.st;
  const int tid = threadIdx.x;
  uint64_t lo = cmin, hi = ~0ull, base = 0;
  Sel out;
  out.ok = false;
  out.c = 0;
  out.incl = 0;
  for (int round = 0; round < 12; round++) {
    const int sh = bucket_shift(hi - lo);
    for (int i = tid; i < NBK; i += NT2) {
      st.bcnt[i] = 0;
      st.bsum[i] = 0;
    }
    bar();
    for_rescan<DT>(
        L, B, R, ws, row,
        [&](int, uint64_t cmp, int rr, uint32_t mu) {
          if (rr != r || cmp < lo || cmp > hi) return;
          const int b = NBK - 1 - (int)((cmp - lo) >> sh);
          atomicAdd(&st.bcnt[b], 1u);
          atomicAdd(&st.bsum[b], by_mass ? (unsigned long long)mu : 1ull);
        },
        [](int) {});
    bar();
    crossing_bucket(L, base, target);
    const int hb = st.si[4];
    if (hb < 0) return out;
    base = st.u0;
    const int nb = st.si[5];
    const uint64_t bl = lo + ((uint64_t)(NBK - 1 - hb) << sh);
    const uint64_t span = (1ull << sh) - 1;
    const uint64_t bh = hi - bl <= span ? hi : bl + span;
    bar();
    if (nb <= XN) {
      clear_gather(st);
      bar();
      for_rescan<DT>(
          L, B, R, ws, row,
          [&](int, uint64_t cmp, int rr, uint32_t mu) {
            if (rr != r || cmp < bl || cmp > bh) return;
            const int p = atomicAdd(&st.si[0], 1);
            if (p < XN) {
              L.ec[p] = cmp;
              L.em[p] = mu;
            }
          },
          [](int) {});
      bar();
      const int n = st.si[0];
      bar();
      Sel sel = select_in_bin(L, n, by_mass, target - base);
      if (sel.ok) sel.incl += base;
      return sel;
    }
    lo = bl;
    hi = bh;
  }
  return out;
}

// Count, mantissa sum and smallest comp of row bin r's elements with comp >= cmin that pass keep(cmp), by a rescan of
// the row (for bins beyond XN elements).  Results in st.si[1], st.u0 and st.cC.
template <int DT, typename P>
__device__ __forceinline__ void reduce_rescan(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int r, uint64_t cmin, P keep) {
  RS& st = *L.st;
  if (threadIdx.x == 0) {
    st.si[1] = 0;
    st.u0 = 0;
    st.cC = ~0ull;
  }
  bar();
  for_rescan<DT>(
      L, B, R, ws, row,
      [&](int, uint64_t cmp, int rr, uint32_t mu) {
        if (rr != r || cmp < cmin || !keep(cmp)) return;
        atomicAdd(&st.si[1], 1);
        atomicAdd(&st.u0, (unsigned long long)mu);
        atomicMin(&st.cC, (unsigned long long)cmp);
      },
      [](int) {});
  bar();
}

// Gathers the elements of row bin r with comp >= cmin into L.ec / L.em (any order).  Returns the count, or -1 when
// the bin holds more than XN of them.
template <int DT>
__device__ __forceinline__ int gather_bin(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int r, uint64_t cmin, bool rescan) {
  RS& st = *L.st;
  const int tid = threadIdx.x, G = st.G;
  clear_gather(st);
  bar();
  if (rescan) {
    for_rescan<DT>(
        L, B, R, ws, row,
        [&](int, uint64_t cmp, int rr, uint32_t mu) {
          if (rr != r || cmp < cmin) return;
          const int p = atomicAdd(&st.si[0], 1);
          if (p < XN) {
            L.ec[p] = cmp;
            L.em[p] = mu;
          }
        },
        [](int) {});
  } else {
    // per block, a group of 16 lanes: the word of the bin, searched over the block's words (in rel order; each round
    // loads 16 evenly spaced words and keeps the segment that can hold the bin), then the bin's listed elements (a
    // contiguous run of the block's list), up to 4 per lane per round of loads, appended with one atomic per wave
    {
      const int gl = tid & 15;
      for (int g0 = 0; g0 < G; g0 += NT2 / 16) {  // uniform trip count: the appends are wave-wide
        const int g = g0 + (tid >> 4);
        int eoff = 0, ecnt = 0;
        if (g < G) {
          BH& h = L.bh[g];
          if (gl == 0) h.rs = 0;
          if (h.listed && r >= h.d + h.w0 && r <= h.d + h.w1 && h.n_tab > 0) {
            const uint32_t want = (uint32_t)(r - h.d - h.wt);
            int lo = 0, n = (int)h.n_tab;
            while (n > 1) {
              const int step = (n + 15) >> 4;
              const bool ok = gl * step < n && (word_of(L, ws, row, g, (uint32_t)(lo + gl * step)).x & 0xFFFu) <= want;
              const uint32_t m = (uint32_t)((__ballot(ok) >> (tid & 48)) & 0xFFFFull);
              if (!m) {
                n = 0;
                break;
              }
              const int l = 31 - __clz((int)m);
              lo += l * step;
              n = min(step, n - l * step);
            }
            if (n == 1) {
              const uint4 w = word_of(L, ws, row, g, (uint32_t)lo);
              if ((w.x & 0xFFFu) == want) {
                if (!((w.x >> 12) & 1u)) {  // elements there, not listed: the block is rescanned below
                  if (gl == 0) {
                    h.rs = 1;
                    st.si[3] = 1;
                  }
                } else {
                  eoff = (int)(w.x >> 13);
                  ecnt = (int)w.y;
                }
              }
            }
          }
        }
        const uint64_t* els = g < G ? els_of(ws, G, row, g) + eoff : nullptr;
        for (int k0 = 0; __ballot(k0 < ecnt) != 0ull; k0 += 64) {
          uint64_t c[4];
          uint32_t tk = 0;  // bit j: element k0 + gl + 16 j is taken
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int k = k0 + gl + 16 * j;
            c[j] = k < ecnt ? els[k] : 0ull;
          }
#pragma unroll
          for (int j = 0; j < 4; j++) tk |= (k0 + gl + 16 * j < ecnt && c[j] >= cmin) ? 1u << j : 0u;
          const int nt = __popc(tk);
          const int inc = wave_scan_incl<int>(nt);
          int wb = 0;
          if (lane_id() == 63 && inc) wb = atomicAdd(&st.si[0], inc);
          int p = readlane<int>(wb, 63) + inc - nt;
#pragma unroll
          for (int j = 0; j < 4; j++) {
            if ((tk >> j) & 1u) {
              if (p < XN) {
                L.ec[p] = c[j];
                L.em[p] = weigh(tval(okey_val(comp_key(c[j])), st.K), L.ts).mu;
              }
              p++;
            }
          }
        }
      }
    }
    bar();
    // the blocks that hold unlisted elements of the bin: rescanned (the staging region is reused: words from global)
    for (int g = 0; g < G && st.si[3]; g++) {
      if (!L.bh[g].rs) continue;
      using BL = Blk<DT, NT2>;
      float x[BL::EPT];
      load_block<DT>(L, B, R, ws, row, g, x);
      if (tid == 0) st.wstaged = 0;
#pragma unroll
      for (int e = 0; e < BL::EPT; e++) {
        if (x[e] == -INFINITY) continue;
        const W w = weigh(tval(x[e], st.K), L.ts);
        if (st.row_top - w.bin() != r) continue;
        const uint64_t cmp = comp(okey(x[e]), (uint32_t)(g * BLK + BL::local(e)));
        if (cmp < cmin) continue;
        const int p = atomicAdd(&st.si[0], 1);
        if (p < XN) {
          L.ec[p] = cmp;
          L.em[p] = w.mu;
        }
      }
      bar();
    }
  }
  bar();
  const int n = st.si[0];
  bar();
  return n > XN ? -1 : n;
}

// Adds mass m (< 2^104) into row bin r while the bins are built: its bits below 40 into mlo, the rest into mhi (two
// independent atomics, no carry to propagate; scan_bins recombines them).
__device__ inline void add_bin(const KL& L, int r, u128 m) {
  atomicAdd(&L.mlo[r], (unsigned long long)m & M40);
  atomicAdd(&L.mhi[r], (unsigned long long)(m >> 40));
}
__device__ inline u128 bin_mass(const KL& L, int r) { return ((u128)L.mhi[r] << 40) + L.mlo[r]; }

// Builds the row-bin arrays: masses, counts and the difference array of blocks pinning each bin.  Fast path: from the
// records (exact at bins every block pins).  Fallback: from rescans (exact everywhere).
template <int DT>
__device__ __forceinline__ void build_bins(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, bool rescan) {
  RS& st = *L.st;
  const int tid = threadIdx.x, G = st.G;
  for (int r = tid; r <= L.rhi; r += NT2) {
    L.mlo[r] = 0;
    L.mhi[r] = 0;
    L.cnt[r] = 0;
    L.good[r] = 0;
  }
  if (tid == 0) L.good[L.rhi + 1] = 0;  // the difference array's entries past rhi + 1 are written, never read
  bar();
  if (rescan) {
    for_rescan<DT>(
        L, B, R, ws, row,
        [&](int, uint64_t, int r, uint32_t mu) {
          add_bin(L, r, rw1(mu, r));
          atomicAdd(&L.cnt[r], 1u);
        },
        [](int) {});
    if (tid == 0) L.good[0] = G;  // every bin is exact
    bar();
    return;
  }
  // every listed block's bin words into the row bins; 16 lanes per block, whose window totals are summed in
  // registers; then the block's last lane adds its good intervals and the lumps above and below its window
  {
    constexpr int KW = 4;
    const int gl = tid & 15;
    for (int g = tid >> 4; g < G; g += NT2 / 16) {
      const BH& h = L.bh[g];
      u128 wm = 0;
      uint32_t wc = 0;
      if (h.listed) {
        for (int k0 = 0; k0 < (int)h.n_tab; k0 += 16 * KW) {
          uint4 wv[KW];
#pragma unroll
          for (int kk = 0; kk < KW; kk++) {
            const int k = k0 + gl + kk * 16;
            if (k < (int)h.n_tab) wv[kk] = word_of(L, ws, row, g, (uint32_t)k);
          }
#pragma unroll
          for (int kk = 0; kk < KW; kk++) {
            const int k = k0 + gl + kk * 16;
            if (k >= (int)h.n_tab) continue;
            const int r = h.d + h.wt + (int)(wv[kk].x & 0xFFFu);
            if (r >= NR) continue;
            const uint32_t cn = wv[kk].y;
            const u128 m = rw(((unsigned long long)wv[kk].w << 32) | wv[kk].z, r);
            add_bin(L, r, m);
            atomicAdd(&L.cnt[r], cn);
            wm += m;
            wc += cn;
          }
        }
      }
      wm = row16_scan_incl<u128>(wm);
      wc = row16_scan_incl<uint32_t>(wc);
      if (gl == 15) {
        auto good_iv = [&](int a, int b) {
          a = max(a, 0);
          b = min(b, NR - 1);
          if (a > b) return;
          atomicAdd(&L.good[a], 1);
          atomicSub(&L.good[b + 1], 1);
        };
        if (!h.active) {
          good_iv(0, NR - 1);
        } else {
          good_iv(0, h.d + h.rel_max - 1);
          if (h.listed) good_iv(h.d + h.w0, h.d + h.w1);
          good_iv(h.d + h.rel_min + 1, NR - 1);
          const u128 T = ld128(st.Tlo[g], st.Thi[g]), A = ld128(st.Alo[g], st.Ahi[g]);
          if (h.listed && h.w0 > 0 && (A != 0 || st.nA[g])) {
            const int r = h.d + h.w0 - 1;
            add_bin(L, r, A);
            atomicAdd(&L.cnt[r], st.nA[g]);
          }
          const u128 Bm = h.listed ? T - A - wm : T;
          const uint32_t nB = h.listed ? st.nT[g] - st.nA[g] - wc : st.nT[g];
          if (Bm != 0 || nB) {
            const int r = min(h.d + h.rel_min, NR - 1);
            add_bin(L, r, Bm);
            atomicAdd(&L.cnt[r], nB);
          }
        }
      }
    }
  }
  bar();
}

// Inclusive prefixes over the row bins [0, rhi] (mass, count, pinning blocks): each thread a run of PR bins.
__device__ __forceinline__ void scan_bins(const KL& L) {
  // counts (< 2^24) and pinning-block counts (0..64, as a difference array: partial sums wrap mod 256 and come out
  // exact) share one u32; one exchange serves both scans
  constexpr int PRMAX = (NR + NT2 - 1) / NT2;
  const int n = L.rhi + 1;
  const int pr = (n + NT2 - 1) / NT2;
  const int r0 = threadIdx.x * pr, w = wave_id();
  u128 ms = 0;
  uint32_t ps = 0;
#pragma unroll
  for (int k = 0; k < PRMAX; k++) {
    const int r = r0 + k;
    if (k < pr && r < n) {
      ms += bin_mass(L, r);
      ps += L.cnt[r] + ((uint32_t)L.good[r] << 24);
    }
  }
  const u128 sa = wave_scan_incl_u128(ms);
  const uint32_t sb = wave_scan_incl<uint32_t>(ps);
  bar();
  if (lane_id() == 63) {
    L.red[w] = sa;
    L.redu[w] = sb;
  }
  bar();
  u128 mr = sa - ms;
  uint32_t pv = sb - ps;
  for (int i = 0; i < w; i++) {
    mr += L.red[i];
    pv += L.redu[i];
  }
#pragma unroll
  for (int k = 0; k < PRMAX; k++) {
    const int r = r0 + k;
    if (k < pr && r < n) {
      mr += bin_mass(L, r);
      pv += L.cnt[r] + ((uint32_t)L.good[r] << 24);
      L.mlo[r] = (unsigned long long)mr;
      L.mhi[r] = (unsigned long long)(mr >> 64);
      L.cnt[r] = pv & 0xFFFFFFu;
      L.good[r] = (int)(pv >> 24);
    }
  }
  bar();
}

// The draw inside block g from its listed elements, without a rescan: when every kept element of the block lies in
// its window's listed bins from the block's best on (no mass above the window) and there are at most 64 of them,
// wave 0 loads them, weighs them as the row does, ranks them by index and finds the one whose kept-mass interval
// (index order) holds the local target tl.  Their summed weight must equal the block's kept mass K[g]; otherwise,
// or when the conditions fail, returns -2 (the caller rescans the block).  Ends with a barrier; the result is
// uniform.
__device__ __forceinline__ int draw_listed(const KL& L, char* ws, int row, int g, u128 tl) {
  RS& st = *L.st;
  const BH& h = L.bh[g];
  if (threadIdx.x == 0) st.si[7] = -2;
  bar();
  const bool maybe = h.listed && h.mode != 0 && ld128(st.Alo[g], st.Ahi[g]) == 0 && h.n_tab <= 256;
  if (maybe && wave_id() == 0) {
    const int lane = lane_id();
    const int cR = st.cR;
    // the words of bins up to the cut's: all listed, and how many elements they hold
    bool ok = true;
    uint32_t ne = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int j = lane + 64 * k;
      if (j < (int)h.n_tab) {
        const uint4 w = word_of(L, ws, row, g, (uint32_t)j);
        const int r = h.d + h.wt + (int)(w.x & 0xFFFu);
        if (r <= cR) {
          ok = ok && ((w.x >> 12) & 1u);
          ne += w.y;
        }
      }
    }
    ok = __ballot(!ok) == 0ull;
    ne = wave_sum<uint32_t>(ne);
    if (ok && ne <= 64u) {
      uint64_t cmp = 0, wgt = 0;
      bool kept = false;
      if (lane < (int)ne) {
        cmp = els_of(ws, st.G, row, g)[lane];
        const W w = weigh(tval(okey_val(comp_key(cmp)), st.K), L.ts);
        const int r = st.row_top - w.bin();
        kept = r < NR && (r < cR || (r == cR && cmp >= st.cC));
        wgt = kept ? rw1(w.mu, r) : 0ull;
      }
      const uint32_t idx = comp_idx(cmp);
      int rank = 0;
      for (int u = 0; u < (int)ne; u++) {
        const uint32_t o = __shfl(idx, u);
        const int ok2 = __shfl((int)kept, u);
        rank += (ok2 && o < idx) ? 1 : 0;
      }
      if (kept) {
        L.xs[rank] = idx;
        L.xv[rank] = wgt;
      }
      const int nk = (int)__popcll(__ballot(kept));
      const uint64_t v = lane < nk ? L.xv[lane] : 0ull;
      const u128 incl = wave_scan_incl_u128((u128)v);
      const u128 tot = readlane<u128>(incl, 63);
      if (tot == ld128(st.Klo[g], st.Khi[g])) {
        const bool hit = lane < nk && v != 0 && tl < incl && tl >= incl - v;
        const int l = first_lane(hit);
        if (lane == l) st.si[7] = (int)L.xs[lane];
      }
    }
  }
  bar();
  const int tok = st.si[7];
  bar();
  return tok;
}

// Rescans block g (load_block) and returns the token whose kept-mass interval (index order) holds the local target tl,
// or -1.  The processed block is staged in LDS in token order, so that thread t owns the
// contiguous tokens [t * EPT, t * EPT + EPT): one block scan of the per-thread kept masses finds the thread whose
// interval holds tl, and that thread walks its tokens.
template <int DT>
__device__ __forceinline__ int draw_in_block(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, int g, u128 tl) {
  using BL = Blk<DT, NT2>;
  constexpr int EPT = BL::EPT;
  static_assert(EPT % 4 == 0, "whole float4 runs per thread");
  const RS& st = *L.st;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  float x[EPT];
  float* xs = (float*)L.big;
  if (threadIdx.x == 0) L.st->si[7] = -1;
  load_block<DT>(L, B, R, ws, row, g, x, true);  // the processed block in xs, token order
  const int t0 = (int)threadIdx.x * EPT;
  // kept weight of token t0 + k (-inf clamps to t = -2^30: a bin far past any cut, weight 0); the comp is needed
  // only in the cut's bin
  const int cR = st.cR;
  const unsigned long long cC = st.cC;
  auto kept_w = [&](float v, int k) -> uint64_t {
    const W ww = weigh(tval(v, st.K), L.ts);
    const int r = st.row_top - ww.bin();  // >= 0; cR <= NR
    bool keep = r < cR;
    if (r == cR) keep = r < NR && comp(okey(v), (uint32_t)(lo + t0 + k)) >= cC;  // cR == NR: no cut, bin NR weighs nothing
    return keep ? rw1(ww.mu, r) : 0ull;
  };
#pragma unroll
  for (int k = 0; k < EPT; k += 4) {
    const float4 v = *(const float4*)(xs + t0 + k);
    x[k] = v.x;
    x[k + 1] = v.y;
    x[k + 2] = v.z;
    x[k + 3] = v.w;
  }
  uint64_t wv[EPT], sum = 0;  // at most EPT weights below 2^59 each
#pragma unroll
  for (int k = 0; k < EPT; k++) {
    wv[k] = kept_w(x[k], k);
    sum += wv[k];
  }
  u128 tot;
  const u128 c0 = block_scan_incl_u128<NWV2>((u128)sum, L.red, &tot) - sum;
  if (sum && c0 <= tl && tl < c0 + sum) {
    const uint64_t t = (uint64_t)(tl - c0);  // < sum < 2^63
    uint64_t c = 0;
    int hit = -1;
#pragma unroll
    for (int k = 0; k < EPT; k++) {
      if (hit < 0 && wv[k] && t < c + wv[k]) hit = k;
      c += wv[k];
    }
    L.st->si[7] = lo + t0 + hit;
  }
  bar();
  const int tok = L.st->si[7];
  bar();
  return tok;
}

// The row from the prepared bins.  Returns false when a boundary is not pinned (fast path) or a boundary bin holds
// more than XN elements.
template <int DT>
__device__ __forceinline__ bool resolve_row(const KL& L, const qws_batch& B, const qws_row& R, char* ws, int row, bool rescan, RowRes* rres) {
  RS& st = *L.st;
  const int tid = threadIdx.x, G = st.G;
  int cR = NR;
  uint64_t cC = 0;
  u128 S = Cm(L, NR - 1);
  uint32_t Nk = Cn(L, NR - 1);
  int n = 0;  // elements gathered for the cut's bin
  // ---- min_p: keep t >= t_cut (the kept elements of the bin are not ordered by anything but t)
  if (R.min_p > 0.0f) {
    const float tcut = (float)((double)(st.tmax / 1024.0f) + R.log2_min_p) * 1024.0f;
    const int rm = max(st.row_top - (((int)floorf(tcut)) >> 4), 0);
    if (rm < NR) {
      if (!rescan && !Good(L, rm)) return false;
      n = gather_bin<DT>(L, B, R, ws, row, rm, 0, rescan);
      if (n < 0 && !rescan) return false;
      if (n < 0) {  // a bin beyond XN elements: the kept part by a rescan
        const float Kr = st.K;
        reduce_rescan<DT>(L, B, R, ws, row, rm, 0, [=](uint64_t cmp) { return tval(okey_val(comp_key(cmp)), Kr) >= tcut; });
      } else {
        if (tid == 0) {
          st.si[1] = 0;
          st.u0 = 0;
          st.cC = ~0ull;
        }
        bar();
        uint32_t k = 0;
        uint64_t m = 0, cmin = ~0ull;
        for (int i = tid; i < n; i += NT2) {
          if (tval(okey_val(comp_key(L.ec[i])), st.K) >= tcut) {
            k++;
            m += L.em[i];
            cmin = L.ec[i] < cmin ? L.ec[i] : cmin;
          }
        }
        if (k) {
          atomicAdd(&st.si[1], (int)k);
          atomicAdd(&st.u0, (unsigned long long)m);
          atomicMin(&st.cC, (unsigned long long)cmin);
        }
        bar();
      }
      cR = rm;
      cC = st.cC;
      S = Cm(L, rm - 1) + rw(st.u0, rm);
      Nk = Cn(L, rm - 1) + (uint32_t)st.si[1];
      bar();
    }
  }
  // Kept elements of row bin r (r <= cR): the whole bin above the cut's bin, Nk - Cn(r - 1) in it.  When a boundary
  // falls in a bin all of whose kept elements stay kept, the row bins give its exact count and mass (the bin is good)
  // and the bin is neither gathered nor selected; `whole` then marks a cut's bin kept entirely (cC = 0), whose kept
  // mass per block the bin words give.
  auto kept_in = [&](int r) -> uint32_t { return (r == cR ? Nk : Cn(L, r)) - Cn(L, r - 1); };
  bool whole = false;
  // ---- top-k over the min_p survivors
  if (R.top_k > 0 && Nk > (uint32_t)R.top_k) {
    const int rk = first_cross<false>(L, (u128)(uint32_t)R.top_k);
    if (!rescan && !Good(L, rk)) return false;
    const uint64_t kmin = rk == cR ? cC : 0;
    const uint64_t kt = (uint64_t)(R.top_k - (int)Cn(L, rk - 1));
    if (kept_in(rk) == (uint32_t)kt) {  // the bin's elements all stay, none is selected (Nk > top_k: rk < cR, kmin = 0)
      S = Cm(L, rk);
      cR = rk;
      cC = 0;
      whole = true;
      n = 0;
    } else {
      n = gather_bin<DT>(L, B, R, ws, row, rk, kmin, rescan);
      if (n < 0 && !rescan) return false;
      const Sel sk = n < 0 ? select_rescan<DT>(L, B, R, ws, row, rk, kmin, false, kt) : select_in_bin(L, n, false, kt);
      if (!sk.ok) return false;
      // the mass of the bin's first m elements: a second selection by count gives the element, its mass follows
      if (n < 0) {
        reduce_rescan<DT>(L, B, R, ws, row, rk, sk.c, [](uint64_t) { return true; });
      } else {
        if (tid == 0) st.u0 = 0;
        bar();
        uint64_t m = 0;
        for (int i = tid; i < n; i += NT2)
          if (L.ec[i] >= sk.c) m += L.em[i];
        if (m) atomicAdd(&st.u0, (unsigned long long)m);
        bar();
      }
      cR = rk;
      cC = sk.c;
      S = Cm(L, rk - 1) + rw(st.u0, rk);
      whole = false;
    }
    Nk = (uint32_t)R.top_k;
    bar();
  }
  // ---- top-p over the kept set: the first rank position whose inclusive mass reaches thr
  u128 S2 = S;
  if (R.top_p < 1.0f) {
    const uint64_t TP = (uint64_t)floor((double)R.top_p * 4294967296.0);
    u128 thr = mul_shr_ceil(S, TP, 32);
    if (thr == 0) thr = 1;
    const int rp = first_cross<true>(L, thr);
    if (!rescan && !Good(L, rp)) return false;
    const uint64_t pmin = rp == cR ? cC : 0;
    if (kept_in(rp) == 1u) {  // one kept element in the bin: it reaches thr
      if (rp != cR) {
        S2 = Cm(L, rp);
        whole = true;
        n = 0;
      }
      cR = rp;
      cC = pmin;
    } else {
      n = gather_bin<DT>(L, B, R, ws, row, rp, pmin, rescan);
      if (n < 0 && !rescan) return false;
      const u128 base = Cm(L, rp - 1);
      const int sh = D_EXP - (rp >> 6);
      const u128 need = ((thr - base) + (((u128)1 << sh) - 1)) >> sh;  // the bin's mantissa sum must reach this
      const uint64_t ndc = need > (u128)(~0ull >> 1) ? (~0ull >> 1) : (uint64_t)need;
      const Sel sp = n < 0 ? select_rescan<DT>(L, B, R, ws, row, rp, pmin, true, ndc) : select_in_bin(L, n, true, ndc);
      if (!sp.ok) return false;
      cR = rp;
      cC = sp.c;
      S2 = base + rw(sp.incl, rp);
      whole = false;
    }
  }
  if (tid == 0) {
    st.cR = cR;
    st.cC = cC;
  }
  for (int g = tid; g < G; g += NT2) {
    st.Klo[g] = 0;
    st.Khi[g] = 0;
  }
  bar();
  // ---- kept mass per block (index order) and the block of the draw
  if (rescan) {
    u128 acc = 0;
    for_rescan<DT>(
        L, B, R, ws, row,
        [&](int, uint64_t cmp, int r, uint32_t mu) {
          if (r < cR || (r == cR && cmp >= cC)) acc += rw1(mu, r);
        },
        [&](int g) {
          const u128 s = block_sum_u128<NWV2>(acc, L.red);
          if (threadIdx.x == 0) st128(&st.Klo[g], &st.Khi[g], s);
          acc = 0;
        });
  } else {
    for (int g = tid; g < G; g += NT2) {
      BH& h = L.bh[g];
      int mode = 0;
      if (h.active) {
        if (cR >= NR || cR > h.d + h.rel_min) mode = 2;
        else if (cR < h.d + h.rel_max) mode = 0;
        else mode = 1;  // cR inside the listed window (cR is pinned by every block)
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
    bar();
    {  // the words of mode-1 blocks above the cut's bin (and of the cut's bin when it is kept whole): 16 lanes per
       // block, summed in registers
      constexpr int KW = 4;
      const int rk1 = whole ? cR + 1 : cR;
      const int gl = tid & 15;
      for (int g = tid >> 4; g < G; g += NT2 / 16) {
        const BH& h = L.bh[g];
        if (h.mode != 1) continue;
        u128 km = 0;
        for (int k0 = 0; k0 < (int)h.n_tab; k0 += 16 * KW) {
          uint4 wv[KW];
#pragma unroll
          for (int kk = 0; kk < KW; kk++) {
            const int k = k0 + gl + kk * 16;
            if (k < (int)h.n_tab) wv[kk] = word_of(L, ws, row, g, (uint32_t)k);
          }
#pragma unroll
          for (int kk = 0; kk < KW; kk++) {
            const int k = k0 + gl + kk * 16;
            if (k >= (int)h.n_tab) continue;
            const int r = h.d + h.wt + (int)(wv[kk].x & 0xFFFu);
            if (r < rk1) km += rw(((unsigned long long)wv[kk].w << 32) | wv[kk].z, r);
          }
        }
        km = row16_scan_incl<u128>(km);
        if (gl == 15) atomic_add_u128(&st.Klo[g], &st.Khi[g], km);
      }
    }
    if (cR < NR && !whole) {  // the kept elements of the cut's bin (the last gather) belong to mode-1 blocks
      for (int i = tid; i < n; i += NT2) {
        const uint64_t cmp = L.ec[i];
        if (cmp < cC) continue;
        const int g = (int)(comp_idx(cmp) / BLK);
        atomic_add_u128(&st.Klo[g], &st.Khi[g], rw1(L.em[i], cR));
      }
    }
  }
  bar();
  const uint32_t u24 = draw_u24(R.seed, R.position, R.stream, R.row_key, R.draw_word);
  const u128 tt = mul_shr_floor(S2, u24, 24);
  if (wave_id() == 0) {  // lane g: block g's kept-mass interval
    const int lane = lane_id();
    const u128 k = lane < G ? ld128(st.Klo[lane], st.Khi[lane]) : (u128)0;
    const u128 incl = wave_scan_incl_u128(k);
    const bool hit = lane < G && k != 0 && tt < incl && tt >= incl - k;
    const int l = first_lane(hit);
    if (lane == l) {
      st.si[2] = lane;
      st128(&st.t_lo, &st.t_hi, tt - (incl - k));
    }
    if (l == 64 && lane == 0) st.si[2] = -1;
  }
  bar();
  const int gs = st.si[2];
  const u128 tl = ld128(st.t_lo, st.t_hi);
  bar();
  int tok = -1;
  if (gs >= 0) {
    tok = rescan ? -2 : draw_listed(L, ws, row, gs, tl);
    if (tok == -2) tok = draw_in_block<DT>(L, B, R, ws, row, gs, tl);
  }
  if (B.out_probs) {  // dense probabilities of the kept set (test-hook path), by rescans
    const double S2d = (double)(uint64_t)(S2 >> 64) * 18446744073709551616.0 + (double)(uint64_t)S2;
    for_rescan<DT>(
        L, B, R, ws, row,
        [&](int, uint64_t cmp, int r, uint32_t mu) {
          if (r < cR || (r == cR && cmp >= cC)) B.out_probs[(size_t)row * B.V + comp_idx(cmp)] = (float)((double)rw1(mu, r) / S2d);
        },
        [](int) {});
  }
  if (tid == 0) {
    B.out_tokens[row] = tok;
    if (B.out_info) B.out_info[row] = rescan ? 1 : 0;
    if (rres) {
      RowRes o;
      o.s_lo = (unsigned long long)S2;
      o.s_hi = (unsigned long long)(S2 >> 64);
      o.cC = cC;
      o.cR = cR;
      o.row_top = st.row_top;
      o.K = st.K;
      o.kind = RR_SAMPLED;
      o.tok = tok;
      o.pad = 0;
      rres[row] = o;
    }
  }
  return true;
}

template <int DT>
__global__ void __launch_bounds__(NT2) k_resolve(qws_batch B, int G, char* ws, RowRes* rres) {
  __shared__ unsigned long long s_mlo[NR], s_mhi[NR];
  __shared__ uint32_t s_cnt[NR];
  __shared__ int s_good[NR + 1];
  __shared__ uint64_t s_xs[64], s_xv[64];
  __shared__ uint64_t s_ec[XN];
  __shared__ uint32_t s_em[XN];
  __shared__ __attribute__((aligned(16))) uint32_t s_big[BLK];
  __shared__ int s_nt;
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
  L.xs = s_xs;
  L.xv = s_xv;
  L.ec = s_ec;
  L.em = s_em;
  L.big = s_big;
  L.nt = &s_nt;
  L.ts = s_ts;
  L.bh = s_bh;
  L.st = &s_st;
  L.red = s_red;
  L.redu = s_redu;
  L.red64 = s_red64;
  L.rhi = NR - 1;
  RS& st = s_st;
  const int row = blockIdx.x, tid = threadIdx.x, lane = lane_id();
  const qws_row R = B.rows[row];
  for (int i = tid; i < 512; i += NT2) ((uint4*)s_ts)[i] = ((const uint4*)EXP2_TS)[i];
  // ---- round 1: every block header into LDS, and the first WPF bin words of every block into registers (words
  // past a block's count are loaded and dropped)
  constexpr int WPF = 32, PW = MAXG * WPF / NT2;
  static_assert(PW * NT2 == MAXG * WPF && WPF <= CAP, "prefetched words");
  uint4 pw[PW];
#pragma unroll
  for (int k = 0; k < PW; k++) {
    const int i = tid + k * NT2, g = i / WPF;
    pw[k] = g < G ? ((const uint4*)(rec_of(ws, G, row, g) + TAB_OFF))[i % WPF] : make_uint4(0u, 0u, 0u, 0u);
  }
  const bool hstaged = (size_t)G * sizeof(Rec) <= (size_t)BLK * 4;
  const int hstride = hstaged ? (int)sizeof(Rec) : (int)HDR_FIX;
  {
    const int HW = hstride / 16;
    uint4* hs = (uint4*)s_big;
    for (int i = tid; i < G * HW; i += NT2) hs[i] = ((const uint4*)rec_of(ws, G, row, i / HW))[i % HW];
  }
  if (tid == 0) {
    st.G = G;
  }
  bar();
  // the staged header of block g (its fixed fields only unless hstaged)
  auto hdr = [&](int g) -> const Rec& { return *(const Rec*)((const char*)s_big + (size_t)g * hstride); };
  for (int g = tid; g < G; g += NT2) {
    const Rec& H = hdr(g);
    BH h;
    h.max_key = H.max_key;
    h.max_idx = H.max_idx;
    h.flags = H.flags;
    h.c = H.c;
    h.rel_max = H.rel_max;
    h.rel_min = H.rel_min;
    h.w0 = H.w0;
    h.w1 = H.w1;
    h.wt = h.w0;
    h.n_win = (h.flags & RF_WIN) ? H.n_win : 0u;
    h.n_tab = (h.flags & RF_WIN) ? H.n_tab : 0u;
    h.n_patch = (h.flags & RF_CAND) ? H.n_patch : -1;
    h.d = 0;
    h.active = 0;
    h.listed = 0;
    h.mode = 0;
    h.woff = 0;
    h.eoff = 0;
    h.ecnt = 0;
    h.ebase = 0;
    s_bh[g] = h;
  }
  if (tid < 64) {  // the row's best: one wave max over the blocks (G <= 64: lane g wrote block g)
    const uint64_t v = tid < G && (s_bh[tid].flags & RF_CAND) ? comp(s_bh[tid].max_key, s_bh[tid].max_idx) : 0ull;
    const uint64_t m = wave_max_u64(v);
    if (tid == 0) st.best = m;
  }
  bar();
  const uint64_t best = st.best;
  const float K = kscale(R.temperature);
  if (best == 0 || !(R.temperature > 0.0f) || !(K < INFINITY)) {  // no candidate, or a greedy row
    if (tid == 0) {
      B.out_tokens[row] = best == 0 ? 0 : (int)comp_idx(best);
      if (B.out_info) B.out_info[row] = 2;
      if (rres) {
        RowRes o = {};
        o.kind = best == 0 ? RR_EMPTY : RR_GREEDY;
        o.tok = B.out_tokens[row];
        rres[row] = o;
      }
    }
    return;
  }
  if (tid == 0) {
    st.K = K;
    st.tmax = tval(okey_val(comp_key(best)), K);
    st.N = tfloor(st.tmax) >> 10;
    st.row_top = st.N * FB + (FB - 1);
  }
  bar();
  // ---- per block (a thread each): realigned totals and the mass above the window from the block's Horner
  // prefixes: with E = 35 - (N - c), T = P[E] and the mass of the powers of two e < ea = P[ea - 1] * 2^(E - ea + 1)
  for (int g = tid; g < G; g += NT2) {
    BH& h = s_bh[g];
    const Rec& H = hdr(g);
    const Rec& HG = hstaged ? H : *(const Rec*)rec_of(ws, G, row, g);
    u128 T = 0, A = 0;
    uint32_t nT = 0, nA = 0;
    if (h.flags & RF_CAND) {
      const int dn = st.N - h.c;
      const int E = D_EXP - dn;
      const int ea = (h.flags & RF_WIN) ? (h.w0 >> 6) : 0;
      if (E >= 0) {
        T = ((u128)HG.phi[E] << 64) | HG.plo[E];
        nT = HG.pc[E];
        if (ea > 0) {
          const int k = min(ea - 1, E);
          A = shl128_wide(((u128)HG.phi[k] << 64) | HG.plo[k], E - k);
          nA = HG.pc[k];
        }
      }
      if ((h.flags & RF_WIN) && (h.w0 & 63)) {
        const int sh = D_EXP - dn - (h.w0 >> 6);
        if (sh >= 0) {
          A += shl128(H.pmu, sh);
          nA += H.pcnt;
        }
      }
      h.d = dn * FB;
      h.active = h.d + h.rel_max < NR;
      // a usable window lies inside the row window; clip it to the block's occupied bins
      if ((h.flags & RF_WIN) && h.active && h.d + h.w0 < NR && h.w0 <= h.rel_min && h.w1 >= h.rel_max) {
        h.listed = 1;
        if (h.w0 < h.rel_max) {  // nothing lies above the best: the window starts there
          h.w0 = h.rel_max;
          A = 0;
          nA = 0;
        }
        h.w1 = min(h.w1, h.rel_min);
      }
    }
    st128(&st.Tlo[g], &st.Thi[g], T);
    st128(&st.Alo[g], &st.Ahi[g], A);
    st.nT[g] = nT;
    st.nA[g] = nA;
  }
  if (tid < 64) {  // the last row bin any active block adds to (its lowest candidate's)
    const BH& h = s_bh[tid < G ? tid : 0];
    const int v = tid < G && h.active ? min(h.d + h.rel_min, NR - 1) : 0;
    const int m = wave_max_u32((uint32_t)v);
    if (tid == 0) st.rhi = m;
  }
  bar();
  // ---- the listed blocks' bin words into LDS (when they fit): the prefetched ones, then (round 2) the rest
  if (tid < 64) {
    const int c = tid < G && s_bh[tid].listed ? (int)s_bh[tid].n_tab : 0;
    const int inc = wave_scan_incl<int>(c);
    if (tid < G) s_bh[tid].woff = inc - c;
    const bool more = __ballot(c > WPF) != 0ull;
    if (tid == 63) {
      st.nw = inc;
      st.wmore = more ? 1 : 0;
    }
  }
  bar();
  if (tid == 0) st.wstaged = st.nw <= WCAP;
  if (st.nw <= WCAP) {
    uint4* wsd = (uint4*)s_big;
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int i = tid + k * NT2, g = i / WPF, kk = i % WPF;
      if (g < G && s_bh[g].listed && kk < (int)s_bh[g].n_tab) wsd[s_bh[g].woff + kk] = pw[k];
    }
    if (st.wmore) {
      for (int i = tid; i < st.nw; i += NT2) {
        const int g = block_at(L, G, i, [](const BH& h) { return h.woff; });
        const int kk = i - s_bh[g].woff;
        if (kk >= WPF) wsd[i] = ((const uint4*)(rec_of(ws, G, row, g) + TAB_OFF))[kk];
      }
    }
  }
  bar();
  // pass 0 from the records, pass 1 (when pass 0 cannot pin a boundary) from exact rescans of the logits; one
  // expansion of the row's code serves both
  bool done = false;
  for (int pass = (R.test_flags & QWS_TF_RESCAN) ? 1 : 0; pass < 2 && !done; pass++) {
    if (pass == 1) bar();
    L.rhi = pass == 1 ? NR - 1 : st.rhi;
    build_bins<DT>(L, B, R, ws, row, pass == 1);
    scan_bins(L);
    done = resolve_row<DT>(L, B, R, ws, row, pass == 1, rres);
  }
  if (!done && tid == 0) {  // a boundary bin beyond XN elements
    B.out_tokens[row] = -1;
    if (B.out_info) B.out_info[row] = -1;
    if (rres) {
      RowRes o = {};
      o.kind = RR_FAIL;
      o.tok = -1;
      rres[row] = o;
    }
  }
}

}  // namespace qws

// ---------------------------------------------------------------------------------------------- launcher
namespace qws {
// Optional launch timing (profiling only): events recorded around each kernel of qws_sample.  Callers on several
// threads serialise on the mutex while timing is on; with timing off a launch only reads the atomic flag.
struct Timing {
  std::atomic<bool> on{false};
  std::mutex mu;
  int n = 0;
  static constexpr int CAPN = 4096;
  hipEvent_t ev[CAPN][3];
  bool made = false;
};
static Timing g_timing;

int blocks_of(int V) { return (V + BLK - 1) / BLK; }
size_t rows_ws_bytes(int B, int V) { return (size_t)B * blocks_of(V) * REC_BYTES; }

// Compute units of the device that `st` runs on (queried once per device and cached; 256 on MI355X).  Safe under
// concurrent callers: a racing first query stores the same value twice.
int cu_count(hipStream_t st) {
  static std::atomic<int> cus[64];
  int d = -1;
  if (hipStreamGetDevice(st, &d) != hipSuccess && hipGetDevice(&d) != hipSuccess) return 256;
  if (d < 0 || d >= 64) return 256;
  int n = cus[d].load(std::memory_order_relaxed);
  if (!n) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || n <= 0) n = 256;
    cus[d].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <int DT>
static hipError_t launch(const qws_batch& b, int G, char* ws, hipStream_t st, const VerifyIO& v) {
  std::unique_lock<std::mutex> lk(g_timing.mu, std::defer_lock);
  if (g_timing.on.load(std::memory_order_relaxed)) lk.lock();
  const bool tm = lk.owns_lock() && g_timing.on.load(std::memory_order_relaxed) && g_timing.n < Timing::CAPN;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][0], st);
  // a grid within one workgroup per CU (small batches, latency-bound) runs 1,024-thread workgroups: half the
  // elements per thread on each block's chain of phases; larger grids run three 512-thread workgroups per CU
  if (b.B * G <= cu_count(st))
    hipLaunchKernelGGL((k_scan<DT, NT1L>), dim3(b.B * G), dim3(NT1L), 0, st, b, G, ws, v);
  else
    hipLaunchKernelGGL((k_scan<DT, NT1S>), dim3(b.B * G), dim3(NT1S), 0, st, b, G, ws, v);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][1], st);
  hipLaunchKernelGGL((k_resolve<DT>), dim3(b.B), dim3(NT2), 0, st, b, G, ws, v.rres);
  e = hipGetLastError();
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n++][2], st);
  return e;
}

hipError_t launch_rows(const qws_batch& b, int G, char* ws, hipStream_t st, const VerifyIO& v) {
  return b.dtype == QWS_DTYPE_F32 ? launch<QWS_DTYPE_F32>(b, G, ws, st, v) : launch<QWS_DTYPE_BF16>(b, G, ws, st, v);
}
}  // namespace qws

extern "C" int qws_timing(int enable) {
  using namespace qws;
  std::lock_guard<std::mutex> lk(g_timing.mu);
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

extern "C" int qws_timing_read(float* ms_scan, float* ms_resolve, int* launches) {
  using namespace qws;
  std::lock_guard<std::mutex> lk(g_timing.mu);
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
  *ms_scan = a;
  *ms_resolve = r;
  *launches = g_timing.n;
  g_timing.n = 0;
  return 0;
}

// ---------------------------------------------------------------------------------------------- no-allocation entry
// qws_sample_noalloc's workspace: a file-scope device array (each GPU the library runs on holds its own copy until
// the process ends).  Host code never passes `scratch` itself to a kernel (in host code the name is a host-side
// stand-in, not a device address): each device's address comes from hipGetSymbolAddress, taken once per device with
// that device current, and is used everywhere instead.
static __device__ __align__(256) char scratch[QWS_NOALLOC_SCRATCH_BYTES];

namespace qws {
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];  // per device, written once under g_scratch_mu

// The device address of `scratch` on the device that `st` runs on, or null with *err set
static void* scratch_of(hipStream_t st, hipError_t* err) {
  int d = -1;
  if ((*err = hipStreamGetDevice(st, &d)) != hipSuccess) return nullptr;
  if (d < 0 || d >= 64) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[d]) {
    int cur = -1;
    if ((*err = hipGetDevice(&cur)) != hipSuccess) return nullptr;
    if (cur != d && (*err = hipSetDevice(d)) != hipSuccess) return nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != d) (void)hipSetDevice(cur);
    if ((*err = e) != hipSuccess) return nullptr;
    if (!p) {
      *err = hipErrorInvalidSymbol;
      return nullptr;
    }
    g_scratch_ptr[d] = p;
  }
  *err = hipSuccess;
  return g_scratch_ptr[d];
}
}  // namespace qws

extern "C" size_t qws_sample_ws_bytes(int B, int V) {
  if (B < 1 || V < 8) return 0;
  return qws::rows_ws_bytes(B, V);
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
  const VerifyIO none = {nullptr, 0, nullptr, nullptr, nullptr, nullptr, 0, nullptr, nullptr};
  return (int)launch_rows(*b, G, (char*)ws, (hipStream_t)stream, none);
}

namespace qws {
__global__ void k_map_ids(const int* tok, const int* idmap, int Vd, int B, int* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B) return;
  const int t = tok[i];
  out[i] = (t >= 0 && t < Vd) ? idmap[t] : -1;
}
}  // namespace qws

extern "C" int qws_draft_pick(const qws_batch* b, const int* idmap, int* out_ids, void* ws, size_t ws_bytes, void* stream) {
  using namespace qws;
  if (!b || !idmap || !out_ids) return QWS_ERR_INVALID;
  const int e = qws_sample(b, ws, ws_bytes, stream);
  if (e) return e;
  hipLaunchKernelGGL(k_map_ids, dim3((b->B + 255) / 256), dim3(256), 0, (hipStream_t)stream, b->out_tokens, idmap, b->V, b->B, out_ids);
  return (int)hipGetLastError();
}

extern "C" int qws_sample_noalloc(const qws_batch* b, void* stream) {
  using namespace qws;
  if (!b) return QWS_ERR_INVALID;
  if (b->B >= 1 && b->V >= 8 && qws_sample_ws_bytes(b->B, b->V) > (size_t)QWS_NOALLOC_SCRATCH_BYTES) return QWS_ERR_NOT_SUPPORTED;
  hipError_t e = hipSuccess;
  void* ws = scratch_of((hipStream_t)stream, &e);
  if (!ws) return (int)(e != hipSuccess ? e : hipErrorInvalidValue);
  // the records of every block are written before they are read within a call: nothing needs clearing
  return qws_sample(b, ws, (size_t)QWS_NOALLOC_SCRATCH_BYTES, stream);
}
