// qws block loading: one block of BLK tokens of one logits row, held in registers by a workgroup of NTH threads
// (EPT = BLK / NTH tokens per thread), with the request processors applied exactly as the CPU definition
// (oracle/sampler.py, step 1) states them.
#pragma once
#include "qws_device.h"

namespace qws {

__device__ inline float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Thread layout: element e of a thread is token lo + ((e / VEC) * NTH + tid) * VEC + e % VEC, so a thread's
// elements come in increasing token order and every vector load is coalesced across the workgroup.
template <int DT, int NTH>
struct Blk {
  static constexpr int VEC = DT == QWS_DTYPE_F32 ? 4 : 8;  // tokens per 16-byte load
  static constexpr int EPT = BLK / NTH;
  static constexpr int S = EPT / VEC;
  static_assert(EPT % VEC == 0, "whole vectors per thread");
  __device__ static inline int local(int e) { return ((e / VEC) * NTH + (int)threadIdx.x) * VEC + (e % VEC); }

  // Raw logits of block [lo, hi) of `row`: NaN -> -inf, -inf past hi.
  __device__ static inline void load(const qws_batch& B, int row, int lo, int hi, float (&x)[EPT]) {
    const size_t esz = DT == QWS_DTYPE_F32 ? 4 : 2;
    const char* base = (const char*)B.logits + (size_t)row * (size_t)B.row_stride * esz;
#pragma unroll
    for (int s = 0; s < S; s++) {
      const int i0 = lo + (s * NTH + (int)threadIdx.x) * VEC;
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

  // The banned / allowed bitmask: masked tokens become -inf (engine/src/proc.h:40).  A thread's VEC tokens share
  // one mask word (VEC divides 32 and the vectors are VEC-aligned).
  __device__ static inline void mask(const qws_batch& B, const qws_row& R, int lo, int hi, float (&x)[EPT]) {
    if (!R.mask_mode) return;
    const unsigned* mrow = B.masks + (size_t)R.mask_row * (size_t)B.mask_words;
    const uint32_t flip = R.mask_mode == QWS_MASK_ALLOWED ? 0xFFFFFFFFu : 0u;
#pragma unroll
    for (int s = 0; s < S; s++) {
      const int i0 = lo + (s * NTH + (int)threadIdx.x) * VEC;
      if (i0 >= hi) continue;
      const uint32_t mw = mrow[i0 >> 5] ^ flip;
#pragma unroll
      for (int j = 0; j < VEC; j++)
        if ((mw >> ((i0 + j) & 31)) & 1u) x[s * VEC + j] = -INFINITY;
    }
  }
};

// Does the row touch individual tokens (history, drafts, stop ids, bias)?  Masks are applied densely.
__device__ inline bool row_touches(const qws_row& R) {
  return R.proc_on && (R.n_prompt > 0 || R.n_gen > 0 || R.n_drafts > 0 || R.n_bias > 0 || (R.n_stop > 0 && R.min_tokens > R.ngen + R.n_drafts));
}

// Per-block processor state: tab[token - lo] = count | bias slot | stop | prompt (the reference builds the same
// state densely per request, engine/src/proc.cu:72-103; here it is rebuilt per block from the row's lists).  Every
// token touched for the first time is appended to tl (up to TCAP; *nt counts them all).  tab holds BLK words of
// LDS.  Ends with a barrier.
constexpr int TCAP = 1024;  // touched tokens per block processed sparsely
template <int NTH>
__device__ void build_tab(const qws_batch& B, const qws_row& R, int lo, int hi, uint32_t* tab, uint16_t* tl, int* nt) {
  uint4* t4 = (uint4*)tab;
  for (int i = threadIdx.x; i < BLK / 4; i += NTH) t4[i] = make_uint4(0u, 0u, 0u, 0u);
  if (threadIdx.x == 0) *nt = 0;
  __syncthreads();
  auto mark = [&](int j, uint32_t v, bool add) {
    const uint32_t old = add ? atomicAdd(&tab[j], v) : atomicOr(&tab[j], v);
    if (old == 0u) {
      const int p = atomicAdd(nt, 1);
      if (p < TCAP) tl[p] = (uint16_t)j;
    }
  };
  const int* h = B.hist + R.hist_off;
  for (int j = threadIdx.x; j < R.n_prompt; j += NTH) {
    const int id = h[j];
    if (id >= lo && id < hi) mark(id - lo, TB_PROMPT, false);
  }
  for (int j = threadIdx.x; j < R.n_gen; j += NTH) {
    const int id = h[R.n_prompt + j];
    if (id >= lo && id < hi) mark(id - lo, 1u, true);
  }
  for (int j = threadIdx.x; j < R.n_drafts; j += NTH) {
    const int id = B.drafts[R.draft_off + j];
    if (id >= lo && id < hi) mark(id - lo, 1u, true);
  }
  if (R.min_tokens > R.ngen + R.n_drafts) {
    for (int j = threadIdx.x; j < R.n_stop; j += NTH) {
      const int id = B.stop_ids[R.stop_off + j];
      if (id >= lo && id < hi) mark(id - lo, TB_STOP, false);
    }
  }
  for (int j = threadIdx.x; j < R.n_bias; j += NTH) {
    const int id = B.bias_ids[R.bias_off + j];
    if (id >= lo && id < hi) mark(id - lo, (uint32_t)(j + 1) << TB_SLOT_SHIFT, false);
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

// One raw logit (NaN -> -inf) with the row's bitmask applied.
template <int DT>
__device__ inline float raw_masked(const qws_batch& B, const qws_row& R, int row, int i) {
  float x;
  if constexpr (DT == QWS_DTYPE_F32)
    x = ((const float*)B.logits)[(size_t)row * (size_t)B.row_stride + i];
  else
    x = bf16f(((const uint16_t*)B.logits)[(size_t)row * (size_t)B.row_stride + i]);
  x = x != x ? -INFINITY : x;
  if (R.mask_mode) {
    const uint32_t mw = B.masks[(size_t)R.mask_row * (size_t)B.mask_words + (i >> 5)] ^ (R.mask_mode == QWS_MASK_ALLOWED ? 0xFFFFFFFFu : 0u);
    if ((mw >> (i & 31)) & 1u) x = -INFINITY;
  }
  return x;
}

// Loads block [lo, hi) of a row with every processor applied.  The touched tokens are processed sparsely: one
// thread per touched token computes its value into pv and the table word becomes its slot + 1; every other token
// only gets the zero bias (x + 0 turns -0 into +0, as the reference's __fadd_rn(x, 0.0f)).  Beyond TCAP touched
// tokens the table is applied densely.  tab: BLK words of LDS; tl / pv: TCAP entries; nt: an LDS int.
template <int DT, int NTH>
__device__ inline void load_processed(const qws_batch& B, const qws_row& R, int row, int lo, int hi, uint32_t* tab, uint16_t* tl, float* pv, int* nt,
                                      float (&x)[Blk<DT, NTH>::EPT]) {
  using BL = Blk<DT, NTH>;
  BL::load(B, row, lo, hi, x);
  if (!R.proc_on) return;
  BL::mask(B, R, lo, hi, x);
  if (!row_touches(R)) {
#pragma unroll
    for (int e = 0; e < BL::EPT; e++) x[e] = x[e] + 0.0f;
    return;
  }
  build_tab<NTH>(B, R, lo, hi, tab, tl, nt);
  const int n = *nt;
  const float* bias_row = B.bias_vals + R.bias_off;
  if (n <= TCAP) {  // each thread rewrites only the table words of its own touched tokens
    for (int p = threadIdx.x; p < n; p += NTH) {
      const int j = tl[p];
      pv[p] = proc_one(raw_masked<DT>(B, R, row, lo + j), tab[j], R, bias_row);
      tab[j] = (uint32_t)(p + 1);
    }
    __syncthreads();
  }
#pragma unroll
  for (int s = 0; s < BL::S; s++) {
    const uint4* t4 = (const uint4*)(tab + (s * NTH + (int)threadIdx.x) * BL::VEC);
#pragma unroll
    for (int v = 0; v < BL::VEC / 4; v++) {
      const uint4 tv = t4[v];
      const uint32_t tw[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int e = s * BL::VEC + v * 4 + j;
        if (tw[j] == 0u)
          x[e] = x[e] + 0.0f;
        else if (n <= TCAP)
          x[e] = pv[tw[j] - 1];
        else
          x[e] = proc_one(x[e], tw[j], R, bias_row);
      }
    }
  }
  __syncthreads();
}

}  // namespace qws
