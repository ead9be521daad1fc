// qws row results shared by the sampling kernels (qws_sample.hip) and the speculative-verify kernels
// (qws_verify.hip).
#pragma once
#include <atomic>
#include <mutex>

#include "qws_block.h"

namespace qws {

// A resolved row as k_resolve leaves it for the verify kernels.  The kept set is the rank prefix of the candidates
// with a nonzero weight cut at (cR, cC): row bin r = row_top - (q >> 4) < cR, or r == cR and comp(key, index) >= cC
// (cR = NBIN: no cut); S2 = its exact mass in row units (a candidate weighs mu << (D_EXP - (r >> 6))).
struct RowRes {
  unsigned long long s_lo, s_hi;  // S2
  unsigned long long cC;
  int cR, row_top;
  float K;                        // kscale(T)
  int kind;                       // RR_*
  int tok;                        // the row's own draw from p (the greedy token for RR_GREEDY, 0 for RR_EMPTY)
  int pad;
};
enum : int { RR_FAIL = -1, RR_EMPTY = 0, RR_GREEDY = 1, RR_SAMPLED = 2 };

// Extra work of k_scan / k_resolve for the rows of a verify call (all null / 0 for qws_sample).
struct VerifyIO {
  const int* dtok;     // [Bs][K] draft tokens: row b * (K + 1) + t verifies dtok[b * K + t] for t < K
  int K;
  float* vx;           // [Bs * (K + 1)]: the processed value of the verified token, written by the block holding it
  float* vq;           // [Bs * (K + 1)]: the draft's probability of that token (0 outside the draft table), ditto
  const int* inv;      // [V] reduced index of each target id, or -1
  const float* dprob;  // [Bs][K][Vd]
  int Vd;
  RowRes* rres;        // [Bs * (K + 1)]
  const int* nchain;   // [Bs] or null: drafts t >= nchain[b] are delta proposals (q = 1 at the draft)
};

// weight of one mantissa in row bin r (< 2^59: a 64-bit shift)
__device__ inline uint64_t row_weight(uint32_t mu, int r) { return (uint64_t)mu << (D_EXP - (r >> 6)); }

// Optional launch timing (profiling only): HIP events recorded around a call's two kernels (events 0, 1, 2 of a call).
// Callers on several threads serialise on the mutex while timing is on; with timing off a launch only reads the flag.
struct Timing {
  std::atomic<bool> on{false};
  std::mutex mu;
  int n = 0;
  static constexpr int CAPN = 4096;
  hipEvent_t ev[CAPN][3];
  bool made = false;
};
Timing& sample_timing();  // qws_sample's k_scan and k_resolve
Timing& verify_timing();  // qws_verify's k_vres and k_vfin

int blocks_of(int V);
int cu_count(hipStream_t st);  // compute units of the device that st runs on
size_t rows_ws_bytes(int B, int V);  // workspace of k_scan / k_resolve for B rows of V tokens
// k_resolve over b's rows, launched by the translation unit that compiles the instance it launches
typedef hipError_t (*ResolveLaunch)(const qws_batch& b, int G, char* ws, hipStream_t st, RowRes* rres);
// k_scan, then `resolve`
hipError_t launch_rows(const qws_batch& b, int G, char* ws, hipStream_t st, const VerifyIO& v, ResolveLaunch resolve);

}  // namespace qws
