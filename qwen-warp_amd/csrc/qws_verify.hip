// qws speculative verify for MI355X (gfx950): rejection sampling of K draft tokens against K + 1 target rows per
// sequence, with the residual max(0, p - q) resampled on the GPU (engine/src/mtp_sample.cu:227-258 accept_core).
//
// A call verifies Bs sequences in four launches:
//   k_scan, k_resolve  the sampling kernels over the Bs * (K + 1) target rows (row b * (K + 1) + t sees d_1..d_t as
//                      generated tokens): each row's kept set, its exact mass S2 and its own draw from p with the
//                      residual / bonus random word; k_scan also keeps the processed value of the draft each row tests.
//   k_vres   (Bs x G)  the accept tests of a sequence (one lane per row: u * floor(q(d) * S2) < w(d) * 2^24, exact
//                      integers), then, when a draft is rejected, block g's residual mass
//                      sum over kept tokens of max(0, w - floor(q * S2)), q looked up through the inverse id map, and,
//                      when the ending row's own draw from p was left to these kernels, block g's kept mass.
//   k_vfin   (Bs)      picks the block of the residual draw by those masses (or of the draw from p: the bonus row, the
//                      broken-residual control, a residual of zero) and the token inside it by one rescan of that
//                      block (inverse CDF in index order), and writes the emitted tokens.
// k_resolve takes a verify row's own draw from p only when one wave finishes the row (at most 64 candidates); the
// other rows end at S2 (RowRes.tok = -1), since a sequence draws from p at most once, at its ending row.
// The definition is oracle/sampler.py verify_seq.
#include <math.h>

#include "qws_sample.h"

namespace qws {

constexpr int NT3S = 512, NT3L = 1024;   // verify workgroups: 1,024 threads when the grid fits one per CU
constexpr int KMAX = 15;  // drafts per sequence (the reference's widest verify, engine/src/mtp.cu:391)
// A chunk is one wave's part of one stripe of a block at NT3L threads (the tokens of Blk<DT, NT3L>'s slot s of the
// wave's 64 lanes: 64 * VEC consecutive ids), so a block has S * 16 chunks in index order (32 fp32, 16 bf16).
constexpr int NCHMAX = 32;

struct VerifyArgs {
  qws_batch T;               // the target rows
  int Bs, K, Vd, G;
  const int* dtok;           // [Bs][K]
  const float* dprob;        // [Bs][K][Vd]
  const int* inv;            // [V]: reduced index of a target id, or -1
  const RowRes* rres;        // [Bs * (K + 1)]
  const int* nchain;         // [Bs] or null: drafts t >= nchain[b] are delta proposals
  const float* vx;           // [Bs * (K + 1)]
  const float* vq;           // [Bs * (K + 1)]
  unsigned long long* part;  // [Bs][G] x {residual lo, hi, kept lo, hi}: masses of each block of the ending row
  unsigned long long* chunkp;  // [Bs][G][NCHMAX] x {lo, hi}: chunk prefixes of each block (k_vres at NT3L only)
  int chunked;               // k_vres ran at NT3L and wrote chunkp
  int* vs;                   // [Bs]: t* | residual needed << 8
  int* out_tokens;           // [Bs][K + 1]
  int* out_n;                // [Bs]
};

// Inclusive block scans of S values per thread at once (one LDS exchange for all of them): inc[s] = the prefix of value
// s over the threads up to this one, tot[s] = its block total.  red: 68 entries.  Wave 0 turns the wave totals into
// each wave's offset, so a thread reads two words per value, not every wave's total.
template <int NWV, int S>
__device__ inline void block_scans_u128(const u128 (&v)[S], u128* red, u128 (&inc)[S], u128 (&tot)[S]) {
  static_assert(NWV <= 16 && S <= 4, "value s's wave totals in DPP row s of wave 0");
  const int w = wave_id(), lane = lane_id();
#pragma unroll
  for (int s = 0; s < S; s++) inc[s] = wave_scan_incl_u128(v[s]);
  bar();
  if (lane == 63)
#pragma unroll
    for (int s = 0; s < S; s++) red[s * 16 + w] = inc[s];
  bar();
  if (w == 0) {  // lane 16 s + i: wave i's offset within value s; lane 16 s + 15 holds value s's total
    const int s = lane >> 4, i = lane & 15;
    const bool live = s < S && i < NWV;
    const u128 r = live ? red[lane] : (u128)0;
    const u128 x = row16_scan_incl<u128>(r);
    if (live) red[lane] = x - r;
    if (s < S && i == 15) red[64 + s] = x;
  }
  bar();
#pragma unroll
  for (int s = 0; s < S; s++) {
    inc[s] += red[s * 16 + w];
    tot[s] = red[64 + s];
  }
}

// floor(q * S2) exactly for a probability q (NaN and q <= 0 count as 0, q >= 1 as 1); S2 < 2^100
__device__ inline u128 q_fix(float q, u128 S2) {
  if (!(q > 0.0f)) return 0;
  if (q >= 1.0f) return S2;
  const uint32_t b = __float_as_uint(q);
  const int E = (int)(b >> 23);
  const uint32_t m = E ? ((b & 0x7FFFFFu) | 0x800000u) : (b & 0x7FFFFFu);
  return shr128(S2 * (u128)m, E ? 150 - E : 149);  // q = m * 2^-(150 - E), or m * 2^-149 when subnormal
}

__device__ inline u128 s2_of(const RowRes& rr) { return rr.kind == RR_GREEDY ? (u128)1 : (((u128)rr.s_hi << 64) | rr.s_lo); }

// The test of row t of sequence b: returns true when the row ends the sequence (t == K, a row without a sampled
// distribution to test against, or a rejected draft); *rej = a draft was rejected against a sampled row, *flags = the
// row's test flags.  ts: the exp2 table (LDS copy).
__device__ inline bool verify_stop(const VerifyArgs& A, int b, int t, bool* rej, const float2* ts, int* flags) {
  *rej = false;
  const int row = b * (A.K + 1) + t;
  const qws_row R = A.T.rows[row];  // loaded with the row's result, before either is used
  const RowRes rr = A.rres[row];
  *flags = R.test_flags;
  if (t >= A.K || rr.kind == RR_EMPTY || rr.kind == RR_FAIL) return true;
  const int V = A.T.V;
  const int d = A.dtok[b * A.K + t];
  const bool dok = d >= 0 && d < V;
  const u128 S2 = s2_of(rr);
  uint64_t wd = 0;
  if (dok) {
    if (rr.kind == RR_GREEDY) {
      wd = d == rr.tok ? 1u : 0u;
    } else {
      const float x = A.vx[row];
      if (x != -INFINITY) {
        const W w = weigh(tval(x, rr.K), ts);
        const int r = rr.row_top - w.bin();
        if (r < NBIN && (r < rr.cR || (r == rr.cR && comp(okey(x), (uint32_t)d) >= rr.cC))) wd = row_weight(w.mu, r);
      }
    }
  }
  const float qv = dok ? A.vq[row] : 0.0f;  // recorded by the block holding d
  const uint32_t u = draw_u24(R.seed, R.position, R.stream, R.row_key, 0);
  if ((u128)u * q_fix(qv, S2) < ((u128)wd << 24)) return false;  // accept w.p. min(1, p / q)
  *rej = rr.kind == RR_SAMPLED;
  return true;
}

// Residual weights of block g of the rejected row (index layout of Blk<DT, NT3>): kept tokens weigh
// max(0, w - floor(q * S2)); tokens outside the draft table keep w.
// res = false: the kept weights alone (the draw from p), no draft probabilities read.  *kept: the thread's kept weight
// before the residual (< 2^62: EPT <= 16 weights below 2^59 each).
template <int DT, int NT3>
__device__ __forceinline__ void residual_block(const VerifyArgs& A, const qws_row& R, const RowRes& rr, int b, int t, int row, int g, uint32_t* tab,
                                               int* nt, const float2* ts, uint64_t (&wv)[Blk<DT, NT3>::EPT], bool res, uint64_t* kept) {
  using BL = Blk<DT, NT3>;
  constexpr int EPT = BL::EPT;
  const int lo = g * BLK, hi = min(A.T.V, lo + BLK);
  // the inverse map of the block's tokens, loaded before (and together with) the logits
  int iv[EPT];
#pragma unroll
  for (int s = 0; s < BL::S; s++) {
    const int i0 = lo + (s * NT3 + (int)threadIdx.x) * BL::VEC;
#pragma unroll
    for (int v = 0; v < BL::VEC / 4; v++) {
      int4 q4 = make_int4(-1, -1, -1, -1);
      if (i0 < hi) q4 = *(const int4*)(A.inv + i0 + 4 * v);
      iv[s * BL::VEC + 4 * v] = q4.x;
      iv[s * BL::VEC + 4 * v + 1] = q4.y;
      iv[s * BL::VEC + 4 * v + 2] = q4.z;
      iv[s * BL::VEC + 4 * v + 3] = q4.w;
    }
  }
  float x[EPT];
  load_processed<DT, NT3>(A.T, R, row, lo, hi, tab, x, nullptr, nt);
  const u128 S2 = s2_of(rr);
  const float* qrow = A.dprob + ((size_t)b * A.K + t) * A.Vd;
  // a delta proposal (q = 1 at the draft d, 0 elsewhere): the residual is p without d
  const bool delta = A.nchain && t >= A.nchain[b];
  const int dd = delta ? A.dtok[b * A.K + t] : -1;
  // kept weights (cR <= NBIN; the comp is needed only in the cut's bin; -inf shares t = -2^30 with the lower clamp,
  // so it is excluded by value); the exp2 table entries first, in one round of LDS reads
  float tv[EPT];
  float2 te[EPT];
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    tv[e] = tval(x[e], rr.K);
    te[e] = ts[tab_index(tv[e])];
  }
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    const W ww = weigh_e(tv[e], te[e]);
    const int r = rr.row_top - ww.bin();
    bool keep = r < rr.cR && x[e] != -INFINITY;
    if (r == rr.cR) keep = r < NBIN && x[e] != -INFINITY && comp(okey(x[e]), (uint32_t)(lo + BL::local(e))) >= rr.cC;  // cR == NBIN: no cut
    wv[e] = keep ? row_weight(ww.mu, r) : 0ull;
  }
  uint64_t kp = 0;
#pragma unroll
  for (int e = 0; e < EPT; e++) kp += wv[e];
  *kept = kp;
  if (!res) return;  // uniform
  float qv[EPT];  // every gather issued before any is used
  if (delta) {
#pragma unroll
    for (int e = 0; e < EPT; e++) qv[e] = (lo + BL::local(e) == dd) ? 1.0f : 0.0f;
  } else {
#pragma unroll
    for (int e = 0; e < EPT; e++) qv[e] = (wv[e] && iv[e] >= 0 && iv[e] < A.Vd) ? qrow[iv[e]] : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    if (qv[e] > 0.0f) {
      const u128 qf = q_fix(qv[e], S2);
      wv[e] = (u128)wv[e] > qf ? wv[e] - (uint64_t)qf : 0;
    }
  }
}

template <int DT, int NT3>
__global__ void __launch_bounds__(NT3) k_vres(VerifyArgs A) {
  constexpr int NWV3 = NT3 / 64;
  using BL = Blk<DT, NT3>;
  __shared__ __attribute__((aligned(16))) uint32_t s_tab[BLK];
  __shared__ __attribute__((aligned(16))) float2 s_ts[1024];
  __shared__ int s_nt, s_vs;
  __shared__ u128 s_red[68];
  const int b = blockIdx.x / A.G, g = blockIdx.x - b * A.G, tid = threadIdx.x;
  // the exp2 table first: the tests weigh from its LDS copy (no global table read after the rows' loads)
  for (int i = tid; i < 512; i += NT3) ((uint4*)s_ts)[i] = ((const uint4*)EXP2_TS)[i];
  bar();
  if (tid < 64) {  // lane t tests row t; the first row that ends the sequence is t* (lane K always stops)
    bool rej = false;
    int fl = 0;
    const bool stop = tid > A.K || verify_stop(A, b, tid, &rej, s_ts, &fl);
    const int ts = first_lane(stop);
    const bool need = ballot_bit(rej, ts);
    const int flags = readlane<int>(fl, ts);  // row t*'s test flags, loaded by lane t*
    if (tid == 0) {
      s_vs = ts | ((need && !(flags & QWS_TF_BROKEN)) ? 256 : 0);
      if (g == 0) A.vs[b] = s_vs;
    }
  }
  bar();
  const int vs = s_vs;
  const int t = vs & 255, row = b * (A.K + 1) + t;
  const RowRes rr = A.rres[row];
  const bool res = vs & 256, plain = rr.kind == RR_SAMPLED && rr.tok < 0;  // the row's draw from p not taken yet
  if (!res && !plain) return;
  const qws_row R = A.T.rows[row];
  uint64_t wv[BL::EPT], kp;
  residual_block<DT, NT3>(A, R, rr, b, t, row, g, s_tab, &s_nt, s_ts, wv, res, &kp);
  // the weights summed (the residual when the row needs one, else the kept weights) per slot s of the thread, and the
  // kept mass; at NT3L each wave's total of slot s is chunk (s, wave)'s, and the block-cumulative prefix at the end of
  // every chunk goes to chunkp, so that k_vfin rescans one chunk instead of the block
  constexpr int S = NT3 == NT3L ? BL::S : 1;
  static_assert(S + 1 <= 4 && S * NWV3 <= NCHMAX, "chunk layout");
  u128 v[S + 1], inc[S + 1], tot[S + 1];
#pragma unroll
  for (int s = 0; s < S; s++) {
    v[s] = 0;
#pragma unroll
    for (int e = s * (BL::EPT / S); e < (s + 1) * (BL::EPT / S); e++) v[s] += wv[e];
  }
  v[S] = kp;
  block_scans_u128<NWV3, S + 1>(v, s_red, inc, tot);  // the summed weights and the kept mass together
  u128 main = 0;
#pragma unroll
  for (int s = 0; s < S; s++) main += tot[s];
  if (NT3 == NT3L && lane_id() == 63) {
    unsigned long long* cp = A.chunkp + 2 * (((size_t)b * A.G + g) * NCHMAX);
    u128 base = 0;
#pragma unroll
    for (int s = 0; s < S; s++) {
      const u128 P = base + inc[s];
      cp[2 * (s * NWV3 + wave_id())] = (unsigned long long)P;
      cp[2 * (s * NWV3 + wave_id()) + 1] = (unsigned long long)(P >> 64);
      base += tot[s];
    }
  }
  if (tid == 0) {
    unsigned long long* pw = A.part + 4 * ((size_t)b * A.G + g);
    pw[0] = res ? (unsigned long long)main : 0ull;
    pw[1] = res ? (unsigned long long)(main >> 64) : 0ull;
    pw[2] = plain ? (unsigned long long)tot[S] : 0ull;
    pw[3] = plain ? (unsigned long long)(tot[S] >> 64) : 0ull;
  }
}

template <int DT, int NT3>
__global__ void __launch_bounds__(NT3) k_vfin(VerifyArgs A) {
  constexpr int NWV3 = NT3 / 64;
  using BL = Blk<DT, NT3>;
  __shared__ __attribute__((aligned(16))) uint32_t s_tab[BLK];
  __shared__ __attribute__((aligned(16))) float2 s_ts[1024];
  __shared__ int s_nt, s_g, s_c, s_tok, s_plain;
  __shared__ unsigned long long s_tlo, s_thi;
  __shared__ u128 s_red[68];
  constexpr bool CH = NT3 == NT3L;             // chunk prefixes are recorded at NT3L only
  constexpr int NCH = CH ? BL::S * NWV3 : 1;  // chunks per block
  __shared__ u128 s_chp[CH ? MAXG * NCHMAX : 1];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int vs = A.vs[b];
  const int t = vs & 255, row = b * (A.K + 1) + t;
  const RowRes rr = A.rres[row];
  const qws_row R = A.T.rows[row];
  if (tid == 0) {
    s_g = -1;
    s_tok = rr.tok;
    s_plain = 0;
  }
  // the blocks' masses (lane g: block g's) loaded together with the exp2 table
  const int G = A.G;
  u128 kres = 0, kkept = 0;
  if (tid < G) {
    const unsigned long long* pw = A.part + 4 * ((size_t)b * G + tid);
    if (vs & 256) kres = ((u128)pw[1] << 64) | pw[0];
    if (rr.kind == RR_SAMPLED && rr.tok < 0) kkept = ((u128)pw[3] << 64) | pw[2];
  }
  // every block's chunk prefixes (k_vres at NT3L), loaded with the masses and the table
  const bool chunked = CH && A.chunked;
  if (chunked) {
    const unsigned long long* cp = A.chunkp + 2 * ((size_t)b * G * NCHMAX);
    for (int i = tid; i < G * NCH; i += NT3) {
      const int g = i / NCH, c = i - g * NCH;
      const vu4 q = gmem((const vu4*)(cp + 2 * ((size_t)g * NCHMAX + c)))[0];
      s_chp[g * NCHMAX + c] = ((u128)(((unsigned long long)q.w << 32) | q.z) << 64) | (((unsigned long long)q.y << 32) | q.x);
    }
  }
  for (int i = tid; i < 512; i += NT3) ((uint4*)s_ts)[i] = ((const uint4*)EXP2_TS)[i];
  bar();
  if (tid < 64) {  // lane g: block g's interval of the residual (R == 0: of p, as without a residual)
    const uint32_t u = draw_u24(R.seed, R.position, R.stream, R.row_key, R.draw_word);
    u128 Rt = 0;
    int gp = -1;     // the block (wave-uniform)
    u128 tl = 0;     // the target inside it
    bool pl = false;  // the draw from p
    if (vs & 256) {
      const u128 k = kres;
      const u128 incl = wave_scan_incl_u128(k);
      Rt = readlane<u128>(incl, 63);
      if (Rt != 0) {
        const u128 tt = mul_shr_floor(Rt, u, 24);
        const int l = first_lane(tid < G && k != 0 && tt < incl && tt >= incl - k);
        if (l < 64) {
          gp = l;
          tl = tt - readlane<u128>(incl - k, l);
        }
      }
    }
    if (Rt == 0 && rr.kind == RR_SAMPLED && rr.tok < 0) {  // uniform: the row's draw from p, by the blocks' kept masses
      const u128 k = kkept;
      const u128 incl = wave_scan_incl_u128(k);
      const u128 tt = mul_shr_floor(s2_of(rr), u, 24);  // the kept masses sum to S2
      const int l = first_lane(tid < G && k != 0 && tt < incl && tt >= incl - k);
      if (l < 64) {
        gp = l;
        tl = tt - readlane<u128>(incl - k, l);
        pl = true;
      }
    }
    // the chunk of block gp that holds the target: k_vres recorded the prefixes of the weights it summed (the residual
    // when the row needs one, else the kept weights), so a draw from p after a residual of zero rescans the block
    int cp = -1;
    if (chunked && gp >= 0 && (!pl || !(vs & 256))) {  // uniform
      const u128 P = tid < NCH ? s_chp[gp * NCHMAX + tid] : (u128)0;
      const int c = first_lane(tid < NCH && tl < P);
      if (c < NCH) {
        cp = c;
        tl -= c > 0 ? readlane<u128>(P, c - 1) : (u128)0;
      }
    }
    if (tid == 0) {
      s_g = gp;
      s_c = cp;
      s_plain = pl ? 1 : 0;
      s_tlo = (unsigned long long)tl;
      s_thi = (unsigned long long)(tl >> 64);
    }
  }
  bar();
  const int gs = s_g;
  if (CH && gs >= 0 && s_c >= 0) {  // uniform: the token inside chunk s_c of block gs, by the wave that k_vres summed it in
    const int cs = s_c, sc = cs / NWV3, wc = cs - sc * NWV3;
    const bool mine = wave_id() == wc, resid = !s_plain;
    const int lo = gs * BLK, hi = min(A.T.V, lo + BLK);
    const int i0 = lo + (sc * NT3 + tid) * BL::VEC;  // this lane's VEC tokens of slot sc
    int iv[BL::VEC];  // their reduced indices, loaded before the logits
#pragma unroll
    for (int v = 0; v < BL::VEC / 4; v++) {
      int4 q4 = make_int4(-1, -1, -1, -1);
      if (mine && resid && i0 < hi) q4 = *(const int4*)(A.inv + i0 + 4 * v);
      iv[4 * v] = q4.x;
      iv[4 * v + 1] = q4.y;
      iv[4 * v + 2] = q4.z;
      iv[4 * v + 3] = q4.w;
    }
    float x[BL::EPT];
    load_processed<DT, NT3>(A.T, R, row, lo, hi, s_tab, x, nullptr, &s_nt);  // every thread: the block's processing
    if (mine) {  // uniform in the wave
      float xv[BL::VEC];
#pragma unroll
      for (int j = 0; j < BL::VEC; j++) xv[j] = x[j];
#pragma unroll
      for (int s = 1; s < BL::S; s++)
#pragma unroll
        for (int j = 0; j < BL::VEC; j++) xv[j] = s == sc ? x[s * BL::VEC + j] : xv[j];
      // the same weights as residual_block gives these tokens
      const u128 S2 = s2_of(rr);
      const float* qrow = A.dprob + ((size_t)b * A.K + t) * A.Vd;
      const bool delta = A.nchain && t >= A.nchain[b];
      const int dd = delta ? A.dtok[b * A.K + t] : -1;
      float tv[BL::VEC];
      float2 te[BL::VEC];
#pragma unroll
      for (int j = 0; j < BL::VEC; j++) {
        tv[j] = tval(xv[j], rr.K);
        te[j] = s_ts[tab_index(tv[j])];
      }
      uint64_t wv[BL::VEC];
#pragma unroll
      for (int j = 0; j < BL::VEC; j++) {
        const W ww = weigh_e(tv[j], te[j]);
        const int r = rr.row_top - ww.bin();
        bool keep = r < rr.cR && xv[j] != -INFINITY;
        if (r == rr.cR) keep = r < NBIN && xv[j] != -INFINITY && comp(okey(xv[j]), (uint32_t)(i0 + j)) >= rr.cC;
        wv[j] = keep ? row_weight(ww.mu, r) : 0ull;
      }
      if (resid) {
        float qv[BL::VEC];
        if (delta) {
#pragma unroll
          for (int j = 0; j < BL::VEC; j++) qv[j] = (i0 + j == dd) ? 1.0f : 0.0f;
        } else {
#pragma unroll
          for (int j = 0; j < BL::VEC; j++) qv[j] = (wv[j] && iv[j] >= 0 && iv[j] < A.Vd) ? qrow[iv[j]] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < BL::VEC; j++) {
          if (qv[j] > 0.0f) {
            const u128 qf = q_fix(qv[j], S2);
            wv[j] = (u128)wv[j] > qf ? wv[j] - (uint64_t)qf : 0;
          }
        }
      }
      uint64_t sum = 0;  // VEC weights below 2^59 each
#pragma unroll
      for (int j = 0; j < BL::VEC; j++) sum += wv[j];
      const u128 tl = ((u128)s_thi << 64) | s_tlo;
      const u128 inc = wave_scan_incl_u128((u128)sum);
      u128 c0 = inc - sum;
      if (sum != 0 && c0 <= tl && tl < inc) {
#pragma unroll
        for (int j = 0; j < BL::VEC; j++) {
          const u128 c1 = c0 + wv[j];
          if (wv[j] && c0 <= tl && tl < c1) s_tok = i0 + j;
          c0 = c1;
        }
      }
    }
    bar();
  } else if (gs >= 0) {  // the token whose interval of block gs (index order) holds the local target
    uint64_t wv[BL::EPT], kp;
    residual_block<DT, NT3>(A, R, rr, b, t, row, gs, s_tab, &s_nt, s_ts, wv, !s_plain, &kp);
    const u128 tl = ((u128)s_thi << 64) | s_tlo;
    const int lo = gs * BLK;
    // index order: slot s of every thread, then slot s + 1; the S slots' scans share one exchange
    u128 loc[BL::S], inc[BL::S], tot[BL::S];
#pragma unroll
    for (int s = 0; s < BL::S; s++) {
      loc[s] = 0;
#pragma unroll
      for (int j = 0; j < BL::VEC; j++) loc[s] += wv[s * BL::VEC + j];
    }
    block_scans_u128<NWV3, BL::S>(loc, s_red, inc, tot);
    u128 run = 0;
#pragma unroll
    for (int s = 0; s < BL::S; s++) {
      u128 c0 = run + inc[s] - loc[s];
#pragma unroll
      for (int j = 0; j < BL::VEC; j++) {
        const uint64_t w = wv[s * BL::VEC + j];
        const u128 c1 = c0 + w;
        if (w && c0 <= tl && tl < c1) s_tok = lo + BL::local(s * BL::VEC + j);
        c0 = c1;
      }
      run += tot[s];
    }
    bar();
  }
  const int K = A.K;
  for (int j = tid; j <= K; j += NT3) A.out_tokens[(size_t)b * (K + 1) + j] = j < t ? A.dtok[b * K + j] : (j == t ? s_tok : -1);
  if (tid == 0) A.out_n[b] = t + 1;
}

__global__ void k_inv_fill(int* inv, int V) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < V) inv[i] = -1;
}

__global__ void k_inv_scatter(const int* idmap, int Vd, int V, int* inv) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= Vd) return;
  const int id = idmap[j];
  if (id >= 0 && id < V) atomicMax(&inv[id], j);  // a repeated id keeps its largest reduced index
}

// k_resolve over the target rows of a verify call: each ends at S2 unless one wave finishes it (RowRes)
static hipError_t resolve_verify_rows(const qws_batch& b, int G, char* ws, hipStream_t st, RowRes* rres) {
  if (b.dtype == QWS_DTYPE_F32)
    hipLaunchKernelGGL((k_resolve<QWS_DTYPE_F32, true>), dim3(resolve_grid(b.B)), dim3(NT2), 0, st, b, G, ws, rres);
  else
    hipLaunchKernelGGL((k_resolve<QWS_DTYPE_BF16, true>), dim3(resolve_grid(b.B)), dim3(NT2), 0, st, b, G, ws, rres);
  return hipGetLastError();
}

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

struct VLayout {
  size_t rows, rres, vx, vq, rtok, part, chunkp, vs, total;
};
static VLayout vlayout(int Bs, int K, int V) {
  const size_t Bt = (size_t)Bs * (K + 1);
  VLayout L;
  L.rows = 0;
  L.rres = al256(rows_ws_bytes((int)Bt, V));
  L.vx = L.rres + al256(Bt * sizeof(RowRes));
  L.vq = L.vx + al256(Bt * 4);
  L.rtok = L.vq + al256(Bt * 4);
  L.part = L.rtok + al256(Bt * 4);
  L.chunkp = L.part + al256((size_t)Bs * blocks_of(V) * 32);
  L.vs = L.chunkp + al256((size_t)Bs * blocks_of(V) * NCHMAX * 16);
  L.total = L.vs + al256((size_t)Bs * 4);
  return L;
}

}  // namespace qws

extern "C" size_t qws_verify_ws_bytes(int B, int K, int V) {
  if (B < 1 || K < 1 || K > qws::KMAX || V < 8 || (long long)B * (K + 1) > (1ll << 30)) return 0;
  return qws::vlayout(B, K, V).total;
}

extern "C" int qws_verify(const qws_verify_batch* vb, void* ws, size_t ws_bytes, void* stream) {
  using namespace qws;
  if (!vb || !ws) return QWS_ERR_INVALID;
  const qws_batch& T = vb->target;
  const int Bs = vb->B, K = vb->K;
  if (Bs < 1 || K < 1 || K > KMAX || vb->Vd < 1 || (long long)Bs * (K + 1) != T.B) return QWS_ERR_INVALID;
  if (!vb->draft_tokens || !vb->draft_probs || !vb->inv_map || !vb->out_tokens || !vb->out_n) return QWS_ERR_INVALID;
  if (!T.logits || !T.rows || T.V < 8 || (T.V & 7) || (T.row_stride & 7) || T.row_stride < 0) return QWS_ERR_INVALID;
  if (T.row_stride != 0 && T.row_stride < T.V) return QWS_ERR_INVALID;
  if (T.dtype != QWS_DTYPE_F32 && T.dtype != QWS_DTYPE_BF16) return QWS_ERR_INVALID;
  if (((uintptr_t)T.logits & 15) || ((uintptr_t)ws & 255) || ((uintptr_t)vb->inv_map & 15)) return QWS_ERR_INVALID;
  if (T.masks && T.mask_words * 32LL < T.V) return QWS_ERR_INVALID;
  const int G = blocks_of(T.V);
  if (G > 64) return QWS_ERR_NOT_SUPPORTED;
  const VLayout L = vlayout(Bs, K, T.V);
  if (ws_bytes < L.total) return QWS_ERR_INVALID;
  char* w = (char*)ws;
  hipStream_t st = (hipStream_t)stream;
  qws_batch tb = T;
  tb.out_tokens = (int*)(w + L.rtok);
  VerifyIO io = {vb->draft_tokens, K, (float*)(w + L.vx), (float*)(w + L.vq), vb->inv_map, vb->draft_probs, vb->Vd, (RowRes*)(w + L.rres),
                 vb->n_chain};
  hipError_t e = launch_rows(tb, G, w, st, io, resolve_verify_rows);
  if (e != hipSuccess) return (int)e;
  VerifyArgs A;
  A.T = tb;
  A.Bs = Bs;
  A.K = K;
  A.Vd = vb->Vd;
  A.G = G;
  A.dtok = vb->draft_tokens;
  A.dprob = vb->draft_probs;
  A.inv = vb->inv_map;
  A.rres = io.rres;
  A.nchain = vb->n_chain;
  A.vx = io.vx;
  A.vq = io.vq;
  A.part = (unsigned long long*)(w + L.part);
  A.chunkp = (unsigned long long*)(w + L.chunkp);
  A.vs = (int*)(w + L.vs);
  A.out_tokens = vb->out_tokens;
  A.out_n = vb->out_n;
  // grids within one workgroup per CU (latency-bound) run 1,024-thread workgroups, larger ones 512-thread ones; at
  // 1,024 threads k_vres records chunk prefixes (then Bs <= the CU count, so k_vfin runs 1,024 threads too)
  const bool wide = Bs * G <= cu_count(st);
  A.chunked = wide ? 1 : 0;
  Timing& tg = verify_timing();
  std::unique_lock<std::mutex> lk(tg.mu, std::defer_lock);
  if (tg.on.load(std::memory_order_relaxed)) lk.lock();
  const bool tm = lk.owns_lock() && tg.on.load(std::memory_order_relaxed) && tg.n < Timing::CAPN;
  if (tm) (void)hipEventRecord(tg.ev[tg.n][0], st);
  if (T.dtype == QWS_DTYPE_F32) {
    if (wide)
      hipLaunchKernelGGL((k_vres<QWS_DTYPE_F32, NT3L>), dim3(Bs * G), dim3(NT3L), 0, st, A);
    else
      hipLaunchKernelGGL((k_vres<QWS_DTYPE_F32, NT3S>), dim3(Bs * G), dim3(NT3S), 0, st, A);
    if ((e = hipGetLastError()) != hipSuccess) return (int)e;
    if (tm) (void)hipEventRecord(tg.ev[tg.n][1], st);
    if (Bs <= cu_count(st))
      hipLaunchKernelGGL((k_vfin<QWS_DTYPE_F32, NT3L>), dim3(Bs), dim3(NT3L), 0, st, A);
    else
      hipLaunchKernelGGL((k_vfin<QWS_DTYPE_F32, NT3S>), dim3(Bs), dim3(NT3S), 0, st, A);
  } else {
    if (wide)
      hipLaunchKernelGGL((k_vres<QWS_DTYPE_BF16, NT3L>), dim3(Bs * G), dim3(NT3L), 0, st, A);
    else
      hipLaunchKernelGGL((k_vres<QWS_DTYPE_BF16, NT3S>), dim3(Bs * G), dim3(NT3S), 0, st, A);
    if ((e = hipGetLastError()) != hipSuccess) return (int)e;
    if (tm) (void)hipEventRecord(tg.ev[tg.n][1], st);
    if (Bs <= cu_count(st))
      hipLaunchKernelGGL((k_vfin<QWS_DTYPE_BF16, NT3L>), dim3(Bs), dim3(NT3L), 0, st, A);
    else
      hipLaunchKernelGGL((k_vfin<QWS_DTYPE_BF16, NT3S>), dim3(Bs), dim3(NT3S), 0, st, A);
  }
  e = hipGetLastError();
  if (tm) (void)hipEventRecord(tg.ev[tg.n++][2], st);
  return (int)e;
}

extern "C" int qws_verify_map(const int* idmap, int Vd, int V, int* inv_map, void* stream) {
  using namespace qws;
  if (!idmap || !inv_map || Vd < 1 || V < 8 || (V & 7) || ((uintptr_t)inv_map & 15)) return QWS_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_inv_fill, dim3((V + 255) / 256), dim3(256), 0, st, inv_map, V);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(k_inv_scatter, dim3((Vd + 255) / 256), dim3(256), 0, st, idmap, Vd, V, inv_map);
  return (int)hipGetLastError();
}
