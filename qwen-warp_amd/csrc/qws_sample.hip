// qws sampling kernels for MI355X (gfx950).
//
// One call samples B rows of V logits in two launches:
//   k_scan    (B x G workgroups, one per block of 8,192 tokens): one streaming pass over the logits.  It applies the
//             request processors, finds the block's best candidate and builds an exact LDS histogram of the
//             fixed-point weights by fine bin (a = x / T in log2 units, 64 bins per power of two, counted down from
//             the block's best).  Its record holds the exact per-power-of-two counts and mantissa sums, every fine bin
//             down to the deepest one a row cut can reach in the block (count, mantissa sum and, for the bins it lists,
//             the place of their elements), and the elements of a window of bins chosen from the block's own data:
//             its whole top set when that is small (top-k, min-p, peaked rows), else the bins around its own top-p
//             boundary (flat rows), bucketed by bin.
//   k_resolve (B workgroups, one per row): merges the per-power sums into the row's (a power-of-two's mass is exact in
//             row units), finds each cut (min-p, top-k, top-p) first by power of two, then by fine bin from that
//             power's bins of every block, then inside the bin from its elements (listed ones, or a rescan of a block
//             whose window missed the bin), picks the block of the draw by its exact kept mass and draws the token
//             inside it (Philox4x32-10, inverse CDF in index order) from one rescan of that block.
// The definition being computed is stated in oracle/sampler.py; the reference it restates is
// engine/src/proc.h:39-49 (processors), engine/src/mtp_sample.cu:122-183 (temperature / min_p / top-k /
// top-p), engine/src/mtp_sample.cu:10-27 (Philox draw) and engine/src/misc.cu:50-111 (argmax).
// The record format and k_resolve are in qws_sample.h.
#include "qws_sample.h"

namespace qws {

// ---------------------------------------------------------------------------------------------- k_scan
template <int DT, int NT1>
__global__ void __launch_bounds__(NT1) __attribute__((amdgpu_waves_per_eu(NT1 != NT1S ? 4 : DT == QWS_DTYPE_BF16 ? 8 : 6))) k_scan(qws_batch B, int G, char* ws, VerifyIO VIO) {
  constexpr int NWV1 = NT1 / 64;
  using BL = Blk<DT, NT1>;
  constexpr int EPT = BL::EPT;
  static_assert(NEXP * 8 <= NT1, "eight threads per power of two");
  // LDS, one array whose regions are reused by phase (38,080 bytes: four workgroups fit a CU's 160 KB):
  //   processors:  the processor table [0, 32768) (rows whose only list is a state slot: the block's values), its
  //                bitmap [32768, 33792), the touched-token list [33792, 37888)
  //   afterwards:  histogram u64[NBIN] [0, 18432) (while it is built, a dummy bin per lane after it, in the list
  //                cursors' space), list cursors u32[NBIN] [18432, 27648), a dummy slot per lane [27648, 28160) for
  //                the listing, per-power counts and sums [28160, 28592); the exp2 table [28672, 36864), which the
  //                listing's element buffer reuses once the histogram is built
  //   throughout:  scalars [37888, 38080)
  constexpr int O_CUR = NBIN * 8, O_DUM = O_CUR + NBIN * 4, O_ECNT = O_DUM + 64 * 8, O_EMU = O_ECNT + NEXP * 4;
  constexpr int O_TS = 28672, O_BITS = BLK * 4, O_LIST = O_BITS + BLK / 8, LCAP2 = TCAP, O_SMALL = O_LIST + LCAP2 * 4;
  static_assert(O_EMU % 8 == 0 && O_EMU + NEXP * 8 <= O_TS && O_TS + 8192 <= O_SMALL && O_TS % 16 == 0, "LDS regions");
  static_assert(O_BITS >= O_EMU + NEXP * 8 && CAP * 8 <= 8192 && (NBIN + 64) * 8 <= O_DUM && NBIN + 64 <= 0xFFFF, "LDS regions");
  __shared__ __attribute__((aligned(16))) char s_lds[O_SMALL + 192];
  unsigned long long* const s_hist = (unsigned long long*)s_lds;
  float2* const s_ts = (float2*)(s_lds + O_TS);
  uint32_t* const s_ecnt = (uint32_t*)(s_lds + O_ECNT);
  unsigned long long* const s_emu = (unsigned long long*)(s_lds + O_EMU);
  float* const s_redf = (float*)(s_lds + O_SMALL);  // NWV1 <= 16
  uint32_t& s_imin = *(uint32_t*)(s_lds + O_SMALL + 64);
  int& s_nt = *(int*)(s_lds + O_SMALL + 68);
  int& s_relmin = *(int*)(s_lds + O_SMALL + 72);
  int& s_nl = *(int*)(s_lds + O_SMALL + 76);
  int* const s_win = (int*)(s_lds + O_SMALL + 80);  // 8 words
  float* const s_redb = (float*)(s_lds + O_SMALL + 128);  // NWV1 <= 16: wave maxima of the biased tokens' values
  static_assert(NWV1 <= 16, "wave maxima");

  // Workgroups are dispatched to the 8 XCDs round-robin by index: XCD x runs the contiguous range of (row, block)
  // items [x * chunk, (x + 1) * chunk), so a row's blocks share one XCD's L2 (its history ids are fetched once).
  const int total = B.B * G, chunk = scan_chunk(B.B, G);
  const int item = (int)(blockIdx.x % NXCD) * chunk + (int)(blockIdx.x / NXCD);
  if (item >= total) return;  // spare workgroups of the last XCDs (whole workgroups: before any barrier)
  const int row = item / G, g = item - row * G;
  const int lo = g * BLK, hi = min(B.V, lo + BLK);
  const qws_row R = B.rows[row];
  char* rec = rec_of(ws, G, row, g);
  Rec* H = (Rec*)rec;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  static_assert(NT1 >= 512, "one exp2 table word per thread");
  // this thread's word of the exp2 table (stored to LDS after the block maximum): fp32 rows load it with the block;
  // bf16 rows after the processors, still ahead of the maximum (in the 64-VGPR kernel it would be spilled across them)
  vu4 tsv;
  if constexpr (DT == QWS_DTYPE_F32)
    if (tid < 512) tsv = gmem((const vu4*)EXP2_TS)[tid];

  float x[EPT];
  // No final barrier after the processors: the barrier of the block maximum below comes before the histogram's and
  // the exp2 table's writes over the processors' regions (the maximum's own LDS words are the scalars').
  static_assert(LCAP2 >= TCAP, "every block with patches lists its touched tokens");
  load_processed<DT, NT1, true>(B, R, row, lo, hi, (uint32_t*)s_lds, x, (uint2*)(rec + PATCH_OFF), &s_nt, (uint32_t*)(s_lds + O_LIST), LCAP2, false,
                                (uint32_t*)(s_lds + O_BITS));
  if constexpr (DT == QWS_DTYPE_BF16)
    if (tid < 512) tsv = gmem((const vu4*)EXP2_TS)[tid];
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
  // A lower bound of the row's best from its biased tokens: with no penalty that counts tokens, a biased token's
  // processed value is its logit (NaN -> -inf, masked or stop-suppressed -> -inf) plus its bias, one rounding, as
  // proc_one computes it (the ids are distinct).  A block whose best lies more than D_EXP powers of two below that bound
  // weighs nothing in the row (the row's best is at least the bound) and records only its header.
  // (512-thread workgroups only: the grids of more than one round of workgroups, where a stopped workgroup's CU slot
  // goes to the next; the small grids' 1,024-thread workgroups all run at once)
  float blb = -INFINITY;
  const bool stop_on = R.n_stop > 0 && R.min_tokens > R.ngen + R.n_drafts;
  const bool lbrow = NT1 == NT1S && R.proc_on && R.n_bias > 0 && R.repetition == 1.0f && R.presence == 0.0f && R.frequency == 0.0f &&
                     R.temperature > 0.0f && (!stop_on || R.n_stop <= 16);
  if (lbrow) {  // uniform
    for (int j = tid; j < R.n_bias; j += NT1) {
      const int id = gmem(B.bias_ids)[R.bias_off + j];
      if ((unsigned)id >= (unsigned)B.V) continue;
      float v = BL::at(B, R, row, id);
      if (stop_on)
        for (int k = 0; k < R.n_stop; k++)
          if (gmem(B.stop_ids)[R.stop_off + k] == id) v = -INFINITY;
      blb = fmaxf(blb, v + gmem(B.bias_vals)[R.bias_off + j]);
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
  if (B.out_probs) {  // 0 over the block; k_resolve then writes the kept set (a reused buffer keeps nothing stale)
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const int i = lo + BL::local(e);
      if (i < hi) B.out_probs[(size_t)row * B.V + i] = 0.0f;
    }
  }
  // ---- best candidate: the largest value, lowest index
  float mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < EPT; e++) mloc = fmaxf(mloc, x[e]);
  const float mw = wave_max_f(mloc);
  if (lane == 0) s_redf[wave] = mw;
  if (lbrow) {  // uniform
    const float bw = wave_max_f(blb);
    if (lane == 0) s_redb[wave] = bw;
  }
  if (tid == 0) {
    s_imin = 0xFFFFFFFFu;
    s_relmin = 0;
    s_nl = 0;
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
  bool below = false;  // the block's best more than D_EXP powers of two below the biased tokens' bound
  int dlb = 0;         // powers of two from the block's best up to the bound (when below it)
  if (lbrow && samp && M != -INFINITY) {  // uniform
    float L = s_redb[0];
    for (int i = 1; i < NWV1; i++) L = fmaxf(L, s_redb[i]);
    if (L != -INFINITY) dlb = max((tfloor(tval(L, K)) >> 10) - (tfloor(tval(M, K)) >> 10), 0);
    below = dlb > D_EXP;
  }
  if (M == -INFINITY || !samp || below) {
    if (tid == 0) {
      H->max_key = M == -INFINITY ? KEY_NEGINF : okey(M);
      H->max_idx = M == -INFINITY ? 0u : imax;
      H->c = M == -INFINITY || !samp ? 0 : tfloor(tval(M, K)) >> 10;
      H->flags = M == -INFINITY ? 0 : RF_CAND;
      H->nbw = 0;
      H->w0 = 1;
      H->w1 = 0;
      H->wa = -1;
      H->ea = 0;
      H->n_list = 0;
      H->n_patch = n_patch;
    }
    return;
  }
  // ---- exact histogram of the weights by fine bin, top-down from the best's power of two
  if (tid < 512) ((vu4*)s_ts)[tid] = tsv;  // loaded at the start
  const int qm = tfloor(tval(M, K));
  const int c = qm >> 10;
  const int btop = c * FB + (FB - 1);
  const int r0 = btop - (qm >> 4);  // the best's bin: the first occupied one
  unsigned long long* hist = s_hist;
  uint32_t* cursor = (uint32_t*)(s_lds + O_CUR);  // list slot of each listed bin, then its next free slot
  unsigned long long* const dummy_slots = (unsigned long long*)(s_lds + O_DUM);  // the listing's sink
  for (int i = tid; i < NBIN; i += NT1) hist[i] = 0ull;
  bar();
  uint32_t rp[EPT / 2];  // the elements' bins (16 bits each; >= NBIN: outside the weight window)
  // -inf clamps to t = -2^30, as do finite values of x * K at or below -2^30: its bin lies inside the weight window
  // only when the block's best is within the window's depth of the lower clamp (x / T below about -7.4e8)
  const bool ninf_in = btop + (1 << 26) < NBIN;
  if ((NT1 != NT1S || dlb == 0) && !ninf_in) {  // uniform
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      // -inf lies past the window here.  Branch-free: an element outside the window adds into a dummy bin past the
      // histogram, at most its lane's hist[NBIN + lane] (in the list cursors' space, not yet in use; never read), so
      // the table reads and the atomics of all elements pipeline.
      const W w = weigh(tval(x[e], K), s_ts);
      const uint32_t rel = (uint32_t)(btop - w.bin());  // no element lies above the best's bin
      const uint32_t rx = min(rel, (uint32_t)(NBIN + lane));
      atomicAdd(&hist[rx], (1ull << 40) | (unsigned long long)w.mu);
      if (e & 1)
        rp[e >> 1] |= rx << 16;
      else
        rp[e >> 1] = rx;
    }
  } else {
    // below the biased tokens' bound by dlb powers of two: an element at rel >= relmax lies at row bin rel + 64 dlb
    // or deeper (the row's best is at least the bound), past every row's weight window, so it is neither weighed nor
    // counted (whole waves of such elements branch past the table read and the atomic).  With the best near the lower
    // clamp, -inf is skipped by value.
    const uint32_t relmax = (uint32_t)max(NBIN - FB * dlb, 0);
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      const float t = tval(x[e], K);
      const uint32_t rel = (uint32_t)(btop - (tfloor(t) >> 4));
      uint32_t rx = NBIN + lane;
      if (rel < relmax && (!ninf_in || x[e] != -INFINITY)) {
        rx = rel;
        atomicAdd(&hist[rx], (1ull << 40) | (unsigned long long)weigh(t, s_ts).mu);
      }
      if (e & 1)
        rp[e >> 1] |= rx << 16;
      else
        rp[e >> 1] = rx;
    }
  }
  bar();
  // ---- exact counts and mantissa sums per power of two (eight threads per power, eight bins each), and the last
  // occupied bin (s_relmin, 0 before)
  if (tid < NEXP * 8) {
    const int b0 = (tid >> 3) * FB + (tid & 7) * 8;
    uint32_t cn = 0, last = 0;
    unsigned long long mu = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const unsigned long long h = hist[b0 + k];
      cn += (uint32_t)(h >> 40);
      mu += h & M40;
      last = h ? (uint32_t)(b0 + k) : last;
    }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
      cn += (uint32_t)__shfl_xor((int)cn, m);
      const uint32_t lo32 = (uint32_t)__shfl_xor((int)(uint32_t)mu, m), hi32 = (uint32_t)__shfl_xor((int)(uint32_t)(mu >> 32), m);
      mu += ((unsigned long long)hi32 << 32) | lo32;
      last = max(last, (uint32_t)__shfl_xor((int)last, m));
    }
    if ((tid & 7) == 0) {
      s_ecnt[tid >> 3] = cn;
      s_emu[tid >> 3] = mu;
      if (last) atomicMax(&s_relmin, (int)last);
    }
  }
  bar();
  const int r1 = s_relmin;  // the last occupied bin
  const bool topk = R.top_k > 0, topp = R.top_p < 1.0f, minp = R.min_p > 0.0f;
  // ---- wave 0: the bins to write (down to the deepest bin a row cut can reach here: the block's own min-p cut and
  // its own K-th candidate, since the row's are at or above them) and the window of listed bins
  if (wave == 0) {
    int floor_r = NBIN - 1, hard = NBIN - 1;
    if (minp) {
      const float tcut = (float)((double)(tval(M, K) / 1024.0f) + R.log2_min_p) * 1024.0f;
      const int rm = btop - (((int)floorf(tcut)) >> 4);
      if (rm < NBIN) floor_r = hard = max(rm, 0);
    }
    if (topk) {
      hard = min(hard, blk_cross_cnt(hist, s_ecnt, (uint32_t)R.top_k));
      // the block's likely share of the row's top K (the resolver checks that its window holds the row's cut)
      const uint32_t kk = R.top_k <= 64 ? (uint32_t)R.top_k : (uint32_t)min(R.top_k, 2 * R.top_k / G + 64);
      floor_r = min(floor_r, blk_cross_cnt(hist, s_ecnt, kk));
    }
    floor_r = min(floor_r, r1);
    int w0 = 1, w1 = 0, wa = -1, ea = 0;
    // power-level inclusive prefixes: counts (exact) and approximate masses (relative to the block's top power); when
    // floor_r is the last occupied bin the block's totals cover it
    const uint32_t pcn = lane < NEXP ? s_ecnt[lane] : 0u;
    const float pms = lane < NEXP ? ldexpf((float)s_emu[lane], -lane) : 0.0f;
    const uint32_t icn = wave_scan_incl<uint32_t>(pcn);
    const float ims = wave_scan_incl<float>(pms);
    const bool at_last = floor_r == r1;
    // inclusive prefix of the bin counts over [a, b] into P (the list cursors' space, written only after the window
    // is chosen; wave 0 alone writes and reads it); returns b - a + 1
    uint32_t* P = cursor;
    auto prefix_counts = [&](int a, int b) {
      constexpr int PR = (2 * MARGIN + 64) / 64;  // rounds of 64 bins for the widest span (2 MARGIN + 1 bins)
      const int span = b - a + 1;
      uint32_t cv[PR];  // every count read before the scans
#pragma unroll
      for (int r = 0; r < PR; r++) cv[r] = r * 64 + lane < span ? (uint32_t)(hist[a + r * 64 + lane] >> 40) : 0u;
      uint32_t carry = 0;
#pragma unroll
      for (int r = 0; r < PR; r++) {
        if (r * 64 < span) {  // uniform
          const uint32_t inc = wave_scan_incl<uint32_t>(cv[r]) + carry;
          if (r * 64 + lane < span) P[r * 64 + lane] = inc;
          carry = readlane<uint32_t>(inc, 63);
        }
      }
      return span;
    };
    bool slots_done = false;  // the list slots already written (a flat top-p window, from the shrink's prefix)
    uint32_t slots_n = 0;
    if (topk || topp || minp) {
      const uint32_t nf = at_last ? readlane<uint32_t>(icn, NEXP - 1) : blk_cnt_to(hist, s_ecnt, floor_r);
      if (nf <= (uint32_t)CAP) {  // the whole top set
        w0 = 0;
        w1 = floor_r;
        wa = floor_r;
        ea = floor_r + 1;
      } else {
        int a = 0, b = -1, tp = -1;
        uint32_t budget = (uint32_t)CAP;
        if (topp) {
          // the block's own top-p boundary bp (mass crossing) and the bin t1 before its (CTOP + 1)-th candidate, both
          // from the power-level prefixes above and one fine-bin scan each (independent: issued together)
          const float mf = at_last ? readlane<float>(ims, NEXP - 1) : blk_mass_to(hist, s_emu, floor_r);
          const float tm = R.top_p * mf;
          const uint32_t tc = (uint32_t)CTOP + 1u;  // < nf: pC < NEXP
          const int pP = first_lane(lane < NEXP && ims >= tm), pC = first_lane(lane < NEXP && icn >= tc);
          const unsigned long long hP = pP < NEXP ? hist[pP * FB + lane] : 0ull;
          const float bmP = pP > 0 && pP < NEXP ? readlane<float>(ims, pP - 1) : 0.0f;
          const float fmP = wave_scan_incl<float>(ldexpf((float)(hP & M40), -pP)) + bmP;
          const int bp = min(pP < NEXP ? pP * FB + min(first_lane(fmP >= tm), 63) : NBIN, floor_r);
          // a peaked block also lists its top bins (up to CTOP elements) when they carry a real share of its mass:
          // the row's boundary then lies near the top for a block far below the row's best.  Those elements lie in the
          // powers through pC, so when the (approximate) mass through pC is below the share, the block is not peaked
          // and the fine scans of pC are skipped.
          const bool maybe_peaked = readlane<float>(ims, pC) >= 0.25f * mf;
          unsigned long long hC = 0ull;
          if (maybe_peaked) hC = hist[pC * FB + lane];  // uniform
          const uint32_t bcC = pC > 0 ? readlane<uint32_t>(icn, pC - 1) : 0u;
          const float bmC = pC > 0 ? readlane<float>(ims, pC - 1) : 0.0f;
          const uint32_t fcC = maybe_peaked ? wave_scan_incl<uint32_t>((uint32_t)(hC >> 40)) + bcC : 0u;
          const float fmC = maybe_peaked ? wave_scan_incl<float>(ldexpf((float)(hC & M40), -pC)) + bmC : 0.0f;
          const int fC = min(first_lane(fcC >= tc), 63);
          const int tu = pC * FB + fC - 1, t1 = min(tu, floor_r);
          if (maybe_peaked && t1 >= r0) {
            // mass and count up to t1: when t1 = tu, inside power pC from its fine scans (fC > 0) or all of the powers
            // above pC (fC = 0); a floor below tu takes the general sums
            const bool fast = tu <= floor_r, inC = fC > 0;
            const float m1 = fast ? (inC ? readlane<float>(fmC, fC - 1) : bmC) : blk_mass_to(hist, s_emu, t1);
            if (m1 >= 0.25f * mf) {
              tp = t1;
              budget -= fast ? (inC ? readlane<uint32_t>(fcC, fC - 1) : bcC) : blk_cnt_to(hist, s_ecnt, tp);
            }
          }
          // shrink to the budget, keeping the block's own boundary near the middle: bins leave one at a time from the
          // side farther from bp (the b side on a tie), so the longer side first loses its excess, then the sides
          // alternate starting with b (removed_b(k, D): the bins gone from the b side after k removals, k - that from
          // the a side, D = how many the b side loses first; returned by value, as references into the caller's locals
          // would put them in scratch).  First within MARGIN_FLAT or (peaked) MARGIN_NEAR of bp (one lane per k, the
          // counts' prefix in registers); for a peaked block whose window fits whole, within MARGIN of bp, the b side
          // (below bp) first trimmed to MARGIN_NEAR (the prefix in LDS).  The first window that fits the budget (or is
          // empty) is kept.
          auto removed_b = [](int k, int D) -> int {
            if (D >= 0) return k <= D ? k : D + (k - D + 1) / 2;
            return k - (k <= -D ? k : -D + (k + D) / 2);
          };
          const int mn = tp >= 0 ? MARGIN_NEAR : MARGIN_FLAT;
          a = max(0, bp - mn);
          b = min(floor_r, bp + mn);
          int kk;
          {
            const int span = b - a + 1;  // <= 2 MARGIN_NEAR + 1 < 64
            static_assert(2 * MARGIN_NEAR + 1 < 64 && MARGIN_FLAT <= MARGIN_NEAR, "one lane per k");
            const uint32_t pre = wave_scan_incl<uint32_t>(lane < span ? (uint32_t)(hist[a + lane] >> 40) : 0u);
            const int k = min(lane, span), kb = removed_b(k, (b - bp) - (bp - a)), ka = k - kb;
            const int wa = a + ka, wb = b - kb;
            const uint32_t hi = (uint32_t)__shfl((int)pre, max(wb - a, 0)), lo0 = (uint32_t)__shfl((int)pre, max(ka - 1, 0));
            const uint32_t n = wa > wb ? 0u : hi - (ka > 0 ? lo0 : 0u);
            kk = first_lane(lane <= span && n <= budget);
            const int a0 = a;
            a = readlane<int>(wa, kk);
            b = readlane<int>(wb, kk);
            if (tp < 0 && a <= b) {  // uniform: a flat window [a, b] is listed whole, its slots from the prefix above
              const uint32_t pb = (uint32_t)__shfl((int)pre, max(lane - 1, 0)), c0 = a > a0 ? readlane<uint32_t>(pre, a - a0 - 1) : 0u;
              const int r = a0 + lane;
              if (r >= a && r <= b) cursor[r] = (lane > 0 ? pb : 0u) - c0;
              slots_done = true;
              slots_n = readlane<uint32_t>(pre, b - a0) - c0;
            }
          }
          if (tp >= 0 && kk == 0 && (bp - MARGIN_NEAR > 0 || bp + MARGIN_NEAR < floor_r)) {
            a = max(0, bp - MARGIN);
            b = min(floor_r, bp + MARGIN);
            const int span = prefix_counts(a, b);
            const int D = max(b - bp - MARGIN_NEAR, 0);
            // the elements left after k removals never grow with k, and k = span empties the window: the first k that
            // fits, by two rounds of one k per lane (every s-th k, then the s - 1 before the first that fits)
            auto fits = [&](int k) {
              const int kb = removed_b(k, D), ka = k - kb;
              const int wa = a + ka, wb = b - kb;
              const uint32_t n = wa > wb ? 0u : P[max(wb - a, 0)] - (ka > 0 ? P[ka - 1] : 0u);
              return n <= budget;
            };
            const int s = (span + 62) / 63;  // 63 s >= span: lane 63 tries k = span
            const int k1 = min(lane * s, span);
            const int f1 = min(first_lane(fits(k1)), 63);
            if (f1 == 0) {
              kk = 0;
            } else {
              const int kp = readlane<int>(k1, f1 - 1), kn = readlane<int>(k1, f1);  // fits(kn), not fits(kp)
              const int k2 = kp + 1 + lane;
              kk = kp + 1 + min(first_lane(k2 <= kn && fits(k2)), kn - kp - 1);
            }
            const int kb = removed_b(kk, D), ka = kk - kb;
            a += ka;
            b -= kb;
          }
        } else {  // a min-p / top-k floor with more than CAP tokens above it: the bins just above the floor
          // the first bin from which the bins down to the floor hold at most CAP elements (b + 1: none), first within
          // 2 MARGIN_NEAR bins of the floor, then, when those all fit, within 2 MARGIN
          b = floor_r;
          a = max(0, floor_r - 2 * MARGIN_NEAR);
          int kk;
          {
            const int span = b - a + 1;  // < 64
            const uint32_t pre = wave_scan_incl<uint32_t>(lane < span ? (uint32_t)(hist[a + lane] >> 40) : 0u);
            const uint32_t tot = readlane<uint32_t>(pre, 63), lo0 = (uint32_t)__shfl((int)pre, max(lane - 1, 0));
            const uint32_t n = tot - (lane > 0 ? lo0 : 0u);
            kk = first_lane(lane <= span && (lane == span || n <= (uint32_t)CAP));
            a += kk;
          }
          if (kk == 0 && a > 0) {
            a = max(0, floor_r - 2 * MARGIN);
            const int span = prefix_counts(a, b);
            const uint32_t tot = P[span - 1];
            kk = span;
            for (int k0 = 0; k0 < span; k0 += 64) {  // uniform
              const int k = k0 + lane;
              const uint32_t n = k < span ? tot - (k > 0 ? P[k - 1] : 0u) : 0u;
              const int f = first_lane(k < span && n <= (uint32_t)CAP);
              if (f < 64) {
                kk = k0 + f;
                break;
              }
            }
            a += kk;
          }
        }
        if (tp >= 0) {  // the top part [0, tp], and [a, b] below it (one range when they touch)
          w0 = 0;
          w1 = max(b, tp);
          wa = a <= tp + 1 ? w1 : tp;
          ea = a <= tp + 1 ? w1 + 1 : a;
        } else if (a <= b) {
          w0 = a;
          w1 = b;
          wa = b;
          ea = b + 1;
        }
      }
    }
    // list slots: a prefix of the listed bins' counts, in rel order, over the listed ranges [w0, wa] and [ea, w1] (the
    // bins between them are not listed and get no slot: a peaked block's gap can span hundreds of bins)
    // (four rounds of 64 bins per step, their counts read together: a peaked block's top range can span ~500 bins)
    uint32_t base = slots_n;
    for (int part = 0; part < (slots_done ? 0 : 2); part++) {  // uniform
      const int lo_r = part == 0 ? w0 : max(ea, w0), hi_r = part == 0 ? min(wa, w1) : w1;
      for (int r0c = lo_r; r0c <= hi_r; r0c += 256) {
        uint32_t cn[4];
#pragma unroll
        for (int j = 0; j < 4; j++) cn[j] = r0c + 64 * j + lane <= hi_r ? (uint32_t)(hist[r0c + 64 * j + lane] >> 40) : 0u;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if (r0c + 64 * j > hi_r) break;  // uniform
          const int r = r0c + 64 * j + lane;
          const uint32_t inc = wave_scan_incl<uint32_t>(cn[j]);
          if (r <= hi_r) cursor[r] = base + inc - cn[j];
          base += readlane<uint32_t>(inc, 63);
        }
      }
    }
    if (lane == 0) {
      s_win[0] = w0;
      s_win[1] = w1;
      s_win[2] = wa;
      s_win[3] = ea;
      s_win[4] = (int)base;
      s_win[5] = min(r1, hard) + 1;
      s_nl = 0;
    }
  }
  bar();
  const int w0 = s_win[0], w1 = s_win[1], wa = s_win[2], ea = s_win[3], nbw = s_win[5];
  auto listed = [&](int r) { return r >= w0 && r <= w1 && (r <= wa || r >= ea); };
  // ---- the record: header, per-power sums, bin words (with the list slots of the listed bins)
  if (tid == 0) {
    H->max_key = okey(M);
    H->max_idx = imax;
    H->c = c;
    H->flags = RF_CAND | RF_SAMP;
    H->nbw = nbw;
    H->w0 = w0;
    H->w1 = w1;
    H->wa = wa;
    H->ea = ea;
    H->n_list = s_win[4];
    H->n_patch = n_patch;
  }
  if (tid < NEXP) {
    H->ecnt[tid] = s_ecnt[tid];
    H->emu[tid] = s_emu[tid];
  }

  unsigned long long* BW = (unsigned long long*)(rec + BIN_OFF);
  for (int r = tid; r < nbw; r += NT1) {
    const unsigned long long h = hist[r];
    unsigned long long wd = (h & M40) | ((h >> 40) << 37);
    if (listed(r)) wd |= (1ull << 62) | ((unsigned long long)cursor[r] << 51);
    BW[r] = wd;
  }
  if (w0 <= w1) {
    // elements of the listed bins, bucketed by bin: first compacted into LDS as {value bits, local index} (the exp2
    // table's space, CAP entries; one atomic per wave), then placed one per thread at their bin's next slot
    uint64_t* EL = (uint64_t*)(rec + EL_OFF);
    uint64_t* LW = (uint64_t*)s_ts;  // CAP entries in the exp2 table's space
    auto wave_base = [&](int nw) {  // this lane's first slot in LW: one atomic per wave
      const int inc = wave_scan_incl<int>(nw);
      int wb = 0;
      if (lane == 63 && inc) wb = atomicAdd(&s_nl, inc);
      return readlane<int>(wb, 63) + inc - nw;
    };
    auto rel_of = [&](int e) { return (rp[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu; };  // bin, >= NBIN outside
    if (ea == wa + 1 || wa >= w1) {
      // one range: one test per element (bins below w0 wrap past span; those >= NBIN lie past it), counted, then
      // every element written without a branch, the unlisted ones into the lane's dummy slot (never read)
      const uint32_t span = (uint32_t)(w1 - w0), b0u = (uint32_t)w0;
      int nw = 0;
#pragma unroll
      for (int e = 0; e < EPT; e++) nw += rel_of(e) - b0u <= span ? 1 : 0;
      uint64_t* dst = LW + wave_base(nw);
      uint64_t* dummy = (uint64_t*)(dummy_slots + lane);
#pragma unroll
      for (int e = 0; e < EPT; e++) {
        const bool l = rel_of(e) - b0u <= span;
        *(l ? dst : dummy) = ((uint64_t)__float_as_uint(x[e]) << 32) | (uint32_t)BL::local(e);
        dst += l ? 1 : 0;
      }
    } else if constexpr (DT == QWS_DTYPE_F32) {
      // two ranges, [w0, wa] and [ea, w1] (the second empty when ea > w1): the same two passes with two tests
      // (fp32 only: in the bf16 kernel, at 64 VGPRs, they spill)
      const uint32_t s1 = (uint32_t)(wa - w0), b1 = (uint32_t)w0;
      const uint32_t s2 = ea <= w1 ? (uint32_t)(w1 - ea) : 0u, b2 = ea <= w1 ? (uint32_t)ea : 0xFFFFFFFFu;  // bins < 2^16
      auto in2 = [&](uint32_t r) { return r - b1 <= s1 || r - b2 <= s2; };
      int nw = 0;
#pragma unroll
      for (int e = 0; e < EPT; e++) nw += in2(rel_of(e)) ? 1 : 0;
      uint64_t* dst = LW + wave_base(nw);
      uint64_t* dummy = (uint64_t*)(dummy_slots + lane);
#pragma unroll
      for (int e = 0; e < EPT; e++) {
        const bool l = in2(rel_of(e));
        *(l ? dst : dummy) = ((uint64_t)__float_as_uint(x[e]) << 32) | (uint32_t)BL::local(e);
        dst += l ? 1 : 0;
      }
    } else {
      uint32_t lm = 0;  // bit e: element e is listed
#pragma unroll
      for (int e = 0; e < EPT; e++) {
        lm |= listed((int)rel_of(e)) ? 1u << e : 0u;  // bins >= NBIN lie past w1
      }
      int off = wave_base(__popc(lm));
#pragma unroll
      for (int e = 0; e < EPT; e++)
        if ((lm >> e) & 1u) LW[off++] = ((uint64_t)__float_as_uint(x[e]) << 32) | (uint32_t)BL::local(e);
    }
    bar();
    const int nl = s_nl;
    for (int i = tid; i < nl; i += NT1) {
      const uint64_t lw = LW[i];
      const float v = __uint_as_float((uint32_t)(lw >> 32));
      const int rel = btop - (tfloor(tval(v, K)) >> 4);
      const uint32_t slot = atomicAdd(&cursor[rel], 1u);
      if (slot < (uint32_t)CAP) EL[slot] = comp(okey(v), (uint32_t)lo + (uint32_t)lw);  // always: the window fits the list
    }
  }
}

}  // namespace qws

// ---------------------------------------------------------------------------------------------- launcher
namespace qws {
static Timing g_timing, g_vtiming;
Timing& sample_timing() { return g_timing; }
Timing& verify_timing() { return g_vtiming; }

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

// k_resolve over the rows of qws_sample (the verify rows' k_resolve is launched from qws_verify.hip)
static hipError_t resolve_sample_rows(const qws_batch& b, int G, char* ws, hipStream_t st, RowRes*) {
  if (b.dtype == QWS_DTYPE_F32)
    hipLaunchKernelGGL((k_resolve<QWS_DTYPE_F32, false>), dim3(resolve_grid(b.B)), dim3(NT2), 0, st, b, G, ws, nullptr);
  else
    hipLaunchKernelGGL((k_resolve<QWS_DTYPE_BF16, false>), dim3(resolve_grid(b.B)), dim3(NT2), 0, st, b, G, ws, nullptr);
  return hipGetLastError();
}

template <int DT>
static hipError_t launch(const qws_batch& b, int G, char* ws, hipStream_t st, const VerifyIO& v, ResolveLaunch resolve) {
  std::unique_lock<std::mutex> lk(g_timing.mu, std::defer_lock);
  if (g_timing.on.load(std::memory_order_relaxed)) lk.lock();
  const bool tm = lk.owns_lock() && g_timing.on.load(std::memory_order_relaxed) && g_timing.n < Timing::CAPN;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][0], st);
  // a grid within one workgroup per CU (small batches, latency-bound) runs 1,024-thread workgroups: half the
  // elements per thread on each block's chain of phases; larger grids run three 512-thread workgroups per CU
  if (b.B * G <= cu_count(st))
    hipLaunchKernelGGL((k_scan<DT, NT1L>), dim3(scan_grid(b.B, G)), dim3(NT1L), 0, st, b, G, ws, v);
  else
    hipLaunchKernelGGL((k_scan<DT, NT1S>), dim3(scan_grid(b.B, G)), dim3(NT1S), 0, st, b, G, ws, v);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n][1], st);
  e = resolve(b, G, ws, st, v.rres);
  if (tm) (void)hipEventRecord(g_timing.ev[g_timing.n++][2], st);
  return e;
}

hipError_t launch_rows(const qws_batch& b, int G, char* ws, hipStream_t st, const VerifyIO& v, ResolveLaunch resolve) {
  return b.dtype == QWS_DTYPE_F32 ? launch<QWS_DTYPE_F32>(b, G, ws, st, v, resolve) : launch<QWS_DTYPE_BF16>(b, G, ws, st, v, resolve);
}
}  // namespace qws

namespace qws {
static int timing_enable(Timing& t, int enable) {
  std::lock_guard<std::mutex> lk(t.mu);
  if (enable && !t.made) {
    for (int i = 0; i < Timing::CAPN; i++)
      for (int j = 0; j < 3; j++) {
        const hipError_t e = hipEventCreate(&t.ev[i][j]);
        if (e != hipSuccess) return (int)e;
      }
    t.made = true;
  }
  t.on = enable != 0;
  t.n = 0;
  return 0;
}
static int timing_read(Timing& t, float* ms0, float* ms1, int* launches) {
  if (!ms0 || !ms1 || !launches) return QWS_ERR_INVALID;
  std::lock_guard<std::mutex> lk(t.mu);
  float a = 0.f, r = 0.f;
  for (int i = 0; i < t.n; i++) {
    hipError_t e = hipEventSynchronize(t.ev[i][2]);
    if (e != hipSuccess) return (int)e;
    float x = 0.f, y = 0.f;
    e = hipEventElapsedTime(&x, t.ev[i][0], t.ev[i][1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&y, t.ev[i][1], t.ev[i][2]);
    if (e != hipSuccess) return (int)e;
    a += x;
    r += y;
  }
  *ms0 = a;
  *ms1 = r;
  *launches = t.n;
  t.n = 0;
  return 0;
}
}  // namespace qws

extern "C" int qws_timing(int enable) {
  using namespace qws;
  const int e = timing_enable(g_timing, enable);
  return e ? e : timing_enable(g_vtiming, enable);
}

extern "C" int qws_timing_read(float* ms_scan, float* ms_resolve, int* launches) { return qws::timing_read(qws::g_timing, ms_scan, ms_resolve, launches); }

extern "C" int qws_timing_read_verify(float* ms_accept, float* ms_draw, int* launches) {
  return qws::timing_read(qws::g_vtiming, ms_accept, ms_draw, launches);
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
  return (int)launch_rows(*b, G, (char*)ws, (hipStream_t)stream, none, resolve_sample_rows);
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
  if (!b || !idmap || !out_ids || b->advance) return QWS_ERR_INVALID;  // a draft is not the sequence's token: no step
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
