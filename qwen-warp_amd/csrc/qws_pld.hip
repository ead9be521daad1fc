// qws prompt-lookup (PLD) tail proposer on the device.
//
// The reference proposes the tail of a speculative chain on the host (engine/src/pld.cu, engine/include/pld.h:22-39):
// an n-gram index of the committed history, queried with the last n tokens of history ++ drafts; the engine waits
// on a mapped mailbox for the committed tokens before every proposal (engine/src/mtp.cu:430-437).  Here the
// history lives in HBM next to the sampler's outputs, so appending the tokens a verify call emitted and proposing
// the next tail are two stream-ordered launches with no host round trip.  Instead of a hash index, a proposal scans
// the history from the anchor backwards, 256 positions per step, until it has the `cap` most recent occurrences of
// the query; their backward agreements are measured 64 offsets per wave instruction.  The definition (candidates,
// agreement, ties, gates) is the reference's: oracle/pld.py states it.
#include "qws_pld.h"

namespace qws {

constexpr int NTP = 256;            // workgroup of the proposal kernel
constexpr int PLD_MAXCAP = 4096;    // candidates examined at most (cfg.cap)
constexpr int PLD_OUT = 8;          // proposal slots per row

__global__ void k_pld_reset(void* mem, int max_len, int seq, const int* ctx, int n) {
  int* S = pld_toks(mem, max_len, seq);
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) S[i] = ctx[i];
  if (i == 0) {
    int* h = pld_hdr(mem, max_len, seq);
    h[0] = n;
    h[1] = 0;
  }
}

// Row b appends its tokens up to the first negative one (the -1 after a verify call's emitted tokens).
__global__ void __launch_bounds__(64) k_pld_append(void* mem, int seqs, int max_len, const int* row_seqs, const int* toks, int T) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int seq = row_seqs[b];
  if (seq < 0 || seq >= seqs) return;
  const int t = lane < T ? toks[(size_t)b * T + lane] : -1;
  const unsigned long long neg = __ballot(t < 0);
  pld_append_wave(mem, max_len, seq, t, neg ? __ffsll((long long)neg) - 1 : 64);
}

// One workgroup per row: the proposal for sequence row_seqs[b] after drafts[b][0..nd).
__global__ void __launch_bounds__(NTP) k_pld_propose(void* mem, int seqs, int max_len, qws_pld_cfg c, const int* row_seqs, const int* drafts, int nd,
                                                     int max_tail, int min_len, int* out, int* out_n, int* out_l) {
  __shared__ int s_cand[PLD_MAXCAP];
  __shared__ int s_l[PLD_MAXCAP];
  __shared__ int s_wc[NTP / 64];
  __shared__ int s_best[2];
  const int b = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int seq = row_seqs[b];
  int* o = out + (size_t)b * PLD_OUT;
  if (tid < PLD_OUT) o[tid] = -1;
  const bool ok_seq = seq >= 0 && seq < seqs;
  const int* h = ok_seq ? pld_hdr(mem, max_len, seq) : nullptr;
  const int len = ok_seq && h[1] == 0 ? h[0] : 0;
  const int pa = len - 1, end = pa + nd, n = c.n;
  if (pa < 0 || end + 1 < n) {
    if (tid == 0) {
      out_n[b] = 0;
      out_l[b] = 0;
    }
    return;
  }
  const int* S = pld_toks(mem, max_len, seq);
  const int* D = drafts + (size_t)b * nd;
  auto K = [&](int i) -> int { return i <= pa ? S[i] : D[i - pa - 1]; };
  int key[4];
#pragma unroll
  for (int t = 0; t < 4; t++) key[t] = t < n ? K(end - n + 1 + t) : 0;
  // ---- the `lim` most recent occurrences of the query with j < end, in descending j (engine/src/pld.cu:100-106)
  const int lim = c.longest ? c.cap : 1;
  int found = 0;
  for (int top = min(pa, end - 1); top >= n - 1 && found < lim; top -= NTP) {
    const int j = top - tid;
    bool m = j >= n - 1;
#pragma unroll
    for (int t = 0; t < 4; t++)
      if (t < n) m = m && S[j - n + 1 + t] == key[t];
    const unsigned long long bm = __ballot(m);
    if (lane == 0) s_wc[wave] = __popcll(bm);
    bar();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NTP / 64; w++) {
      before += w < wave ? s_wc[w] : 0;
      total += s_wc[w];
    }
    const int rank = found + before + __popcll(bm & ((1ull << lane) - 1ull));
    if (m && rank < lim) s_cand[rank] = j;
    found += total;
    bar();
  }
  const int nc = min(found, lim);
  // ---- backward agreement of each candidate (engine/src/pld.cu:107-108), one wave per candidate: l = n + the
  // leading equal offsets o = n, n + 1, ... with o < back and j - o >= 0
  for (int ci = wave; ci < nc; ci += NTP / 64) {
    const int j = s_cand[ci];
    int l = -1;
    for (int base = n; l < 0; base += 64) {
      const int ofs = base + lane;
      const bool eq = ofs < c.back && j - ofs >= 0 && K(j - ofs) == K(end - ofs);
      const unsigned long long stop = __ballot(!eq);
      if (stop) l = base + __ffsll((long long)stop) - 1;
    }
    if (lane == 0) s_l[ci] = l;
  }
  bar();
  // ---- the largest agreement, ties to the most recent (engine/src/pld.cu:109-113)
  if (wave == 0) {
    int bl = -1, bc = 0;
    for (int ci = lane; ci < nc; ci += 64) {
      const int l = s_l[ci];
      if (l > bl) {
        bl = l;
        bc = ci;
      }
    }
    // lane order: a larger l wins, then the smaller candidate index (more recent)
    unsigned long long v = bl < 0 ? 0ull : (((unsigned long long)(unsigned)bl << 32) | (unsigned)(PLD_MAXCAP - 1 - bc));
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) {
      const unsigned long long u = __shfl_xor(v, sh);
      v = u > v ? u : v;
    }
    if (lane == 0) {
      s_best[0] = v ? (int)(v >> 32) : -1;
      s_best[1] = v ? PLD_MAXCAP - 1 - (int)(unsigned)(v & 0xFFFFFFFFull) : 0;
    }
  }
  bar();
  const int best_l = s_best[0];
  if (tid == 0) out_l[b] = best_l < 0 ? 0 : best_l;
  if (best_l < 0 || best_l < min_len) {
    if (tid == 0) out_n[b] = 0;
    return;
  }
  const int bj = s_cand[s_best[1]];
  const int ln = min(bj + 1 + max_tail, end + 1) - (bj + 1);
  if (tid < ln) o[tid] = K(bj + 1 + tid);
  if (tid == 0) out_n[b] = ln;
}

}  // namespace qws

extern "C" void qws_pld_default_cfg(qws_pld_cfg* c) {
  c->n = 2;
  c->min_len = 3;
  c->max_tail = 4;
  c->cap = 64;
  c->back = 64;
  c->longest = 1;
}

extern "C" size_t qws_pld_bytes(int seqs, int max_len) {
  if (seqs < 1 || max_len < 1) return 0;
  return (size_t)seqs * qws::pld_stride(max_len);
}

extern "C" int qws_pld_reset(void* mem, int seqs, int max_len, int seq, const int* ctx, int n, void* stream) {
  if (!mem || ((uintptr_t)mem & 255) || seqs < 1 || max_len < 1 || seq < 0 || seq >= seqs || n < 0 || n > max_len || (n > 0 && !ctx))
    return QWS_ERR_INVALID;
  hipLaunchKernelGGL(qws::k_pld_reset, dim3(n > 0 ? (n + 255) / 256 : 1), dim3(256), 0, (hipStream_t)stream, mem, max_len, seq, ctx, n);
  return (int)hipGetLastError();
}

extern "C" int qws_pld_append(void* mem, int seqs, int max_len, const int* row_seqs, int B, const int* toks, int T, void* stream) {
  if (!mem || ((uintptr_t)mem & 255) || seqs < 1 || max_len < 1 || !row_seqs || !toks || B < 0 || T < 1 || T > 64) return QWS_ERR_INVALID;
  if (B == 0) return QWS_OK;
  hipLaunchKernelGGL(qws::k_pld_append, dim3(B), dim3(64), 0, (hipStream_t)stream, mem, seqs, max_len, row_seqs, toks, T);
  return (int)hipGetLastError();
}

extern "C" int qws_pld_propose(void* mem, int seqs, int max_len, const qws_pld_cfg* cfg, const int* row_seqs, int B, const int* drafts, int nd,
                               int max_tail, int min_len, int* out, int* out_n, int* out_l, void* stream) {
  using namespace qws;
  if (!mem || ((uintptr_t)mem & 255) || seqs < 1 || max_len < 1 || !cfg || !row_seqs || B < 0 || nd < 0 || (nd > 0 && !drafts) || !out || !out_n ||
      !out_l || max_tail < 0 || max_tail > PLD_OUT)
    return QWS_ERR_INVALID;
  qws_pld_cfg c = *cfg;  // the reference's clamps (engine/src/pld.cu:56-61)
  c.n = c.n < 1 ? 1 : (c.n > 4 ? 4 : c.n);
  c.max_tail = c.max_tail < 0 ? 0 : (c.max_tail > 7 ? 7 : c.max_tail);
  c.cap = c.cap < 1 ? 1 : c.cap;
  c.back = c.back < 1 ? 1 : c.back;
  c.longest = c.longest ? 1 : 0;
  if (c.longest && c.cap > PLD_MAXCAP) return QWS_ERR_NOT_SUPPORTED;
  if (B == 0) return QWS_OK;
  hipLaunchKernelGGL(k_pld_propose, dim3(B), dim3(NTP), 0, (hipStream_t)stream, mem, seqs, max_len, c, row_seqs, drafts, nd, max_tail, min_len, out,
                     out_n, out_l);
  return (int)hipGetLastError();
}
