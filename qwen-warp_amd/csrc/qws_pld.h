// qws PLD history layout in HBM (qws_pld_*): per sequence a 64-byte header {len, overflow}, then max_len token ids.
#pragma once
#include "qws_device.h"

namespace qws {

constexpr int PLD_HDR = 64;

__host__ __device__ inline size_t pld_stride(int max_len) { return ((size_t)PLD_HDR + (size_t)max_len * 4 + 255) & ~(size_t)255; }
__device__ inline int* pld_hdr(void* mem, int max_len, int seq) { return (int*)((char*)mem + (size_t)seq * pld_stride(max_len)); }
__device__ inline int* pld_toks(void* mem, int max_len, int seq) { return (int*)((char*)mem + (size_t)seq * pld_stride(max_len) + PLD_HDR); }

// One wave appends k <= 64 tokens (lane l holds token l) to sequence seq; tokens beyond max_len mark it overflowed.
__device__ inline void pld_append_wave(void* mem, int max_len, int seq, int t, int k) {
  int* h = pld_hdr(mem, max_len, seq);
  int* S = pld_toks(mem, max_len, seq);
  const int lane = lane_id();
  const int len = h[0];
  const int room = max_len - len;
  const int m = min(k, max(room, 0));
  if (lane < m) S[len + lane] = t;
  if (lane == 0) {
    h[0] = len + m;
    if (k > room) h[1] = 1;
  }
}

}  // namespace qws
