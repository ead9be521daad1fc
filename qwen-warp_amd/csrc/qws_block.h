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

  // Raw logits of block [lo, hi) of `row`, -inf past hi (NaN kept: see fixnan).
  __device__ static inline void load_raw(const qws_batch& B, int row, int lo, int hi, float (&x)[EPT]) {
    const size_t esz = DT == QWS_DTYPE_F32 ? 4 : 2;
    const char* base = (const char*)B.logits + (size_t)row * (size_t)B.row_stride * esz;
#pragma unroll
    for (int s = 0; s < S; s++) {
      const int i0 = lo + (s * NTH + (int)threadIdx.x) * VEC;
      if (i0 < hi) {
        if constexpr (DT == QWS_DTYPE_F32) {
          const vf4 v = *gmem((const vf4*)(base + (size_t)i0 * 4));
          x[s * 4 + 0] = v.x;
          x[s * 4 + 1] = v.y;
          x[s * 4 + 2] = v.z;
          x[s * 4 + 3] = v.w;
        } else {
          const vu4 v = *gmem((const vu4*)(base + (size_t)i0 * 2));
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
  }
  __device__ static inline void fixnan(float (&x)[EPT]) {
#pragma unroll
    for (int e = 0; e < EPT; e++) x[e] = x[e] != x[e] ? -INFINITY : x[e];
  }
  // Raw logits of block [lo, hi) of `row`: NaN -> -inf, -inf past hi.
  __device__ static inline void load(const qws_batch& B, int row, int lo, int hi, float (&x)[EPT]) {
    load_raw(B, row, lo, hi, x);
    fixnan(x);
  }

  // The banned / allowed bitmask: masked tokens become -inf (engine/src/proc.h:40).  A thread's VEC tokens share
  // one mask word (VEC divides 32 and the vectors are VEC-aligned).  mask_words issues the loads of a thread's words
  // (rows with a mask; no lane-dependent branch, so nothing waits for them there: a vector past hi reads the block's
  // last word), apply_mask applies them (nothing for rows without a mask).
  __device__ static inline void mask_words(const qws_batch& B, const qws_row& R, int lo, int hi, uint32_t (&mw)[S]) {
    if (!R.mask_mode) return;  // uniform
    const unsigned* mrow = B.masks + (size_t)R.mask_row * (size_t)B.mask_words;
#pragma unroll
    for (int s = 0; s < S; s++) mw[s] = gmem(mrow)[min(lo + (s * NTH + (int)threadIdx.x) * VEC, hi - 1) >> 5];
  }
  __device__ static inline void apply_mask(const qws_row& R, int lo, int hi, const uint32_t (&mw)[S], float (&x)[EPT]) {
    if (!R.mask_mode) return;  // uniform
    const uint32_t flip = R.mask_mode == QWS_MASK_ALLOWED ? 0xFFFFFFFFu : 0u;
#pragma unroll
    for (int s = 0; s < S; s++) {
      const int i0 = lo + (s * NTH + (int)threadIdx.x) * VEC;
      const uint32_t m = i0 < hi ? (mw[s] ^ flip) >> (i0 & 31) : 0u;
#pragma unroll
      for (int j = 0; j < VEC; j++)
        if ((m >> j) & 1u) x[s * VEC + j] = -INFINITY;
    }
  }
  // Token i (< V) of `row` as load and mask give it: NaN -> -inf, masked -> -inf
  __device__ static inline float at(const qws_batch& B, const qws_row& R, int row, int i) {
    const size_t esz = DT == QWS_DTYPE_F32 ? 4 : 2;
    const char* base = (const char*)B.logits + (size_t)row * (size_t)B.row_stride * esz;
    float v;
    if constexpr (DT == QWS_DTYPE_F32)
      v = *gmem((const float*)(base + (size_t)i * 4));
    else
      v = bf16f(*gmem((const uint16_t*)(base + (size_t)i * 2)));
    v = v != v ? -INFINITY : v;
    if (R.mask_mode) {
      const unsigned* mrow = B.masks + (size_t)R.mask_row * (size_t)B.mask_words;
      const uint32_t flip = R.mask_mode == QWS_MASK_ALLOWED ? 0xFFFFFFFFu : 0u;
      if (((gmem(mrow)[i >> 5] ^ flip) >> (i & 31)) & 1u) v = -INFINITY;
    }
    return v;
  }
};

// ---- device-resident processor state (qws_state_*): per slot, a count word per block (256 bytes), then per block
// BLK entry words {local index (bits 0..12), prompt (bit 13), generated count (bits 16..31)}, one per touched token
constexpr size_t ST_HDR = 256;
constexpr uint32_t SE_LOCAL = 0x1FFFu, SE_PROMPT = 1u << 13;
constexpr int SE_CNT_SHIFT = 16;
constexpr uint32_t SE_CNT_MAX = 0xFFFFu - 64u;  // counts saturate here: drafts (< 64) still fit the table's count field
static_assert(64 * 4 <= ST_HDR, "a count word per block");
__host__ __device__ inline size_t state_slot_bytes(int V) { return ST_HDR + (size_t)((V + BLK - 1) / BLK) * BLK * 4; }
__device__ inline uint32_t* state_counts(void* mem, int V, int slot) { return (uint32_t*)((char*)mem + (size_t)slot * state_slot_bytes(V)); }
__device__ inline uint32_t* state_entries(void* mem, int V, int slot, int g) {
  return (uint32_t*)((char*)mem + (size_t)slot * state_slot_bytes(V) + ST_HDR + (size_t)g * BLK * 4);
}
// the row's state slot, or -1
__device__ inline int row_state(const qws_batch& B, const qws_row& R) {
  return (B.state_mem && R.state_slot >= 0 && R.state_slot < B.state_slots) ? R.state_slot : -1;
}

// Does the row touch individual tokens (history, state, drafts, stop ids, bias)?  Masks are applied densely.
__device__ inline bool row_touches(const qws_batch& B, const qws_row& R) {
  return R.proc_on && (R.n_prompt > 0 || R.n_gen > 0 || R.n_drafts > 0 || R.n_bias > 0 || row_state(B, R) >= 0 ||
                       (R.n_stop > 0 && R.min_tokens > R.ngen + R.n_drafts));
}

// Per-block processor state: tab[token - lo] = count | bias slot | stop | prompt (the reference builds the same
// state densely per request, engine/src/proc.cu:72-103; here it is rebuilt per block from the row's lists).
constexpr int TCAP = 1024;              // processed tokens a block records as patches
constexpr int LCAP = 2048;              // touched tokens of a block processed from a compacted LDS list
constexpr int PF = 8;                   // list entries per thread loaded together with the logits
constexpr uint32_t TB_INC = 1u << 31;   // a list entry that increments the count (otherwise its bits are or-ed)

// The row's token lists as one sequence: prompt ids (flag), generated ids and drafts (counts), stop ids (flag,
// while min_tokens is unmet), bias ids (slot + 1).  Segment ends a <= b <= c <= d <= e.
struct Lists {
  int a, b, c, d, e;
  __device__ explicit Lists(const qws_row& R) {
    a = R.n_prompt;
    b = a + R.n_gen;
    c = b + R.n_drafts;
    d = c + (R.min_tokens > R.ngen + R.n_drafts ? R.n_stop : 0);
    e = d + R.n_bias;
  }
};
// entry j < e: its token id, and in *v the table bits it sets
__device__ inline int list_id(const qws_batch& B, const qws_row& R, const Lists& L, int j, uint32_t* v) {
  if (j < L.b) {
    *v = j < L.a ? TB_PROMPT : TB_INC;
    return gmem(B.hist)[R.hist_off + j];
  }
  if (j < L.c) {
    *v = TB_INC;
    return gmem(B.drafts)[R.draft_off + j - L.b];
  }
  if (j < L.d) {
    *v = TB_STOP;
    return gmem(B.stop_ids)[R.stop_off + j - L.c];
  }
  *v = (uint32_t)(j - L.d + 1) << TB_SLOT_SHIFT;
  return gmem(B.bias_ids)[R.bias_off + j - L.d];
}
// Marks token id in the block's table; with `bits` (BLK / 32 words) also sets its bit there
__device__ inline void mark(uint32_t* tab, uint32_t* bits, int lo, int hi, int id, uint32_t v) {
  if ((unsigned)(id - lo) >= (unsigned)(hi - lo)) return;
  const int l = id - lo;
  if (v & TB_INC)
    atomicAdd(&tab[l], 1u);
  else
    atomicOr(&tab[l], v);
  if (bits) atomicOr(&bits[l >> 5], 1u << (l & 31));
}

// engine/src/proc.h:41-48 on one (already masked) token, one IEEE rounding per operation
__device__ inline float proc_one(float x, uint32_t t, const qws_row& R, const float* bias_row) {
  if (t & TB_STOP) x = -INFINITY;
  const uint32_t slot = (t >> TB_SLOT_SHIFT) & TB_SLOT;
  const float b = slot ? gmem(bias_row)[slot - 1] : 0.0f;
  x = x + b;
  const uint32_t cnt = t & TB_CNT;
  if (R.repetition != 1.0f && ((t & TB_PROMPT) || cnt)) x = x > 0.0f ? x / R.repetition : x * R.repetition;
  if (cnt) {
    x = x - R.frequency * (float)cnt;
    x = x - R.presence;
  }
  return x;
}

// Loads block [lo, hi) of a row with every processor applied (a workgroup of NTH threads; ends with a barrier when
// the row touches tokens).  The first PF list entries of each thread are loaded together with the logits; the
// table is marked with LDS atomics, then each thread applies it to the tokens it holds: touched tokens get
// proc_one.  Every other token keeps its value, -0 included: the reference's zero bias (__fadd_rn(x, 0.0f)) only
// turns -0 into +0, which every consumer here folds the same way (okey, weights, comparisons), and the processed
// logits a caller reads are written as x + 0.
// With `patches` (global, TCAP entries) the processed touched tokens are also recorded there as {local index,
// value} when there are at most TCAP of them; *np (LDS) = the number of touched tokens.  tab: BLK words of LDS.
// list2 (LDS, 3 * lcap2 words apart from tab, or null): when the touched tokens fit there, they are listed while
// other threads still read the table, which saves two barriers.  LB (listed processing; list2 then holds lcap2 words
// and `bits` is BLK / 32 words of LDS): the touched tokens are listed by local index, from a bitmap the marks also
// set (short histories) or from the table words, each is processed by one thread from its word and a second read of
// its logit, and the values go back through the table (no compaction of the owners' values).  Under LB an fp32 row
// whose only list is its state slot (distinct tokens with their counts) takes a shorter form: each entry is processed
// in place in a table of the block's values.  tail = false leaves out the final barrier: the caller
// then orders its next writes to tab (and list2, bits) after a barrier of its own.
template <int DT, int NTH, bool LB = false>
__device__ inline void load_processed(const qws_batch& B, const qws_row& R, int row, int lo, int hi, uint32_t* tab, float (&x)[Blk<DT, NTH>::EPT],
                                      uint2* patches, int* np, uint32_t* list2 = nullptr, int lcap2 = 0, bool tail = true,
                                      uint32_t* bits = nullptr) {
  using BL = Blk<DT, NTH>;
  constexpr int EPT = BL::EPT;
  // every global load of the block is issued before the first wait: logits, mask words, the first list entries
  BL::load_raw(B, row, lo, hi, x);
  if (!R.proc_on) {
    BL::fixnan(x);
    return;
  }
  uint32_t mw[BL::S];
  BL::mask_words(B, R, lo, hi, mw);
  if (!row_touches(B, R)) {
    BL::fixnan(x);
    BL::apply_mask(R, lo, hi, mw, x);
    return;
  }
  const int tid = threadIdx.x;
  const Lists Ls(R);
  // LB: rows whose history takes at most two rounds of loads set bitmap bits as they mark (a second atomic per mark);
  // longer histories list the touched tokens from a scan of the table words instead
  uint32_t* mb = LB && Ls.b <= 2 * PF * NTH ? bits : nullptr;
  const int* hrow = B.hist + R.hist_off;  // prompt then generated ids: entries [0, Ls.b), contiguous
  int pid[PF];
#pragma unroll
  for (int k = 0; k < PF; k++) {
    const int j = tid + k * NTH;
    pid[k] = j < Ls.b ? gmem(hrow)[j] : -1;
  }
  // the block's entries of the row's state slot
  const int sslot = row_state(B, R);
  const uint32_t* sent = nullptr;
  int sn = 0;
  uint32_t se0 = 0;
  if (sslot >= 0) {
    const int g = lo / BLK;
    sn = min((int)gmem(state_counts(B.state_mem, B.V, sslot))[g], BLK);
    sent = state_entries(B.state_mem, B.V, sslot, g);
    if (tid < sn) se0 = gmem(sent)[tid];
  }
  uint4* t4 = (uint4*)tab;
  if constexpr (LB && DT == QWS_DTYPE_F32) {  // (bf16 rows: their 64-register workgroups would spill in the loads)
    if (sslot >= 0 && Ls.e == 0) {
      // State alone: its entries are distinct tokens with their counts, so nothing is marked.  The owners put the
      // block's values in the table (token order), each entry's thread processes its token there, and the owners
      // read the values back: two barriers, no listing, no second read of the logits.
      BL::fixnan(x);
      BL::apply_mask(R, lo, hi, mw, x);
      if (sn == 0) {  // uniform: the slot touches nothing in this block
        if (tid == 0) *np = 0;
        bar();  // *np is read as soon as this returns
        return;
      }
#pragma unroll
      for (int s = 0; s < BL::S; s++)
#pragma unroll
        for (int v = 0; v < BL::VEC / 4; v++) {
          const int e = s * BL::VEC + 4 * v;
          t4[((s * NTH + tid) * BL::VEC) / 4 + v] =
              make_uint4(__float_as_uint(x[e]), __float_as_uint(x[e + 1]), __float_as_uint(x[e + 2]), __float_as_uint(x[e + 3]));
        }
      if (tid == 0) *np = sn;
      bar();
      float* tf = (float*)tab;
      const float* bias_row = B.bias_vals + R.bias_off;
      const bool rec = patches && sn <= TCAP;
      auto entry = [&](int j, uint32_t e) {
        const uint32_t l = e & SE_LOCAL;
        const uint32_t wd = (e >> SE_CNT_SHIFT) | ((e & SE_PROMPT) ? TB_PROMPT : 0u);
        uint2 pt = make_uint2(0xFFFFFFFFu, 0u);  // an entry with nothing to apply: no patch
        if (wd) {
          const float v = proc_one(tf[l], wd, R, bias_row);
          tf[l] = v;
          pt = make_uint2(l, __float_as_uint(v));
        }
        if (rec) patches[j] = pt;
      };
      if (tid < sn) entry(tid, se0);
      for (int j0 = NTH; j0 < sn; j0 += PF * NTH) {
        uint32_t ev[PF];
#pragma unroll
        for (int k = 0; k < PF; k++) {
          const int j = j0 + tid + k * NTH;
          ev[k] = j < sn ? gmem(sent)[j] : 0u;
        }
#pragma unroll
        for (int k = 0; k < PF; k++)
          if (j0 + tid + k * NTH < sn) entry(j0 + tid + k * NTH, ev[k]);
      }
      bar();
#pragma unroll
      for (int s = 0; s < BL::S; s++)
#pragma unroll
        for (int v = 0; v < BL::VEC / 4; v++) {
          const uint4 q = t4[((s * NTH + tid) * BL::VEC) / 4 + v];
          const int e = s * BL::VEC + 4 * v;
          x[e] = __uint_as_float(q.x);
          x[e + 1] = __uint_as_float(q.y);
          x[e + 2] = __uint_as_float(q.z);
          x[e + 3] = __uint_as_float(q.w);
        }
      if (tail) bar();
      return;
    }
  }
  for (int i = tid; i < BLK / 4; i += NTH) t4[i] = make_uint4(0u, 0u, 0u, 0u);
  if (mb && tid < BLK / 128) ((uint4*)mb)[tid] = make_uint4(0u, 0u, 0u, 0u);
  if (tid == 0) *np = 0;
  bar();
#pragma unroll
  for (int k = 0; k < PF; k++) mark(tab, mb, lo, hi, pid[k], tid + k * NTH < Ls.a ? TB_PROMPT : TB_INC);
  // the logits arrived before the first list entries (loads complete in order): NaN and the mask now, so that the
  // mask words die here (a masked touched token still ends -inf: its processed value is read through `at`, or
  // computed in place from the -inf)
  BL::fixnan(x);
  BL::apply_mask(R, lo, hi, mw, x);
  for (int j0 = PF * NTH; j0 < Ls.b; j0 += PF * NTH) {  // the rest of a long history, PF loads in flight per thread
    int id[PF];
#pragma unroll
    for (int k = 0; k < PF; k++) {
      const int j = j0 + tid + k * NTH;
      id[k] = j < Ls.b ? gmem(hrow)[j] : -1;
    }
#pragma unroll
    for (int k = 0; k < PF; k++) mark(tab, mb, lo, hi, id[k], j0 + tid + k * NTH < Ls.a ? TB_PROMPT : TB_INC);
  }
  for (int j = Ls.b + tid; j < Ls.e; j += NTH) {  // drafts, stop ids, bias ids
    uint32_t v;
    const int id = list_id(B, R, Ls, j, &v);
    mark(tab, mb, lo, hi, id, v);
  }
  if (sslot >= 0) {  // state entries: distinct tokens, each adds its count and prompt flag (no other list sets it)
    auto add = [&](uint32_t e) {
      const uint32_t a = (e >> SE_CNT_SHIFT) | ((e & SE_PROMPT) ? TB_PROMPT : 0u);
      if (!a) return;  // nothing to add: the word and the bit stay as they are
      const uint32_t l = e & SE_LOCAL;
      atomicAdd(&tab[l], a);
      if (mb) atomicOr(&mb[l >> 5], 1u << (l & 31));
    };
    if (tid < sn) add(se0);
    for (int j0 = NTH; j0 < sn; j0 += PF * NTH) {
      uint32_t ev[PF];
#pragma unroll
      for (int k = 0; k < PF; k++) {
        const int j = j0 + tid + k * NTH;
        ev[k] = j < sn ? gmem(sent)[j] : 0u;
      }
#pragma unroll
      for (int k = 0; k < PF; k++)
        if (j0 + tid + k * NTH < sn) add(ev[k]);
    }
  }
  bar();
  const float* bias_row = B.bias_vals + R.bias_off;
  if constexpr (LB) {
    // the touched tokens listed: from the bitmap by its first BLK / 32 threads (whole waves), or from each thread's
    // own table words
    static_assert((BLK / 32) % 64 == 0 && BLK / 32 <= NTH, "bitmap words per thread");
    if (mb) {
      if (tid < BLK / 32) {
        uint32_t w = mb[tid];
        const int c = __popc(w);
        const int inc = wave_scan_incl<int>(c);
        int wb = 0;
        if (lane_id() == 63 && inc) wb = atomicAdd(np, inc);
        int p = readlane<int>(wb, 63) + inc - c;
        while (w) {
          const int b = __ffs(w) - 1;
          w &= w - 1u;
          if (p < lcap2) list2[p] = (uint32_t)(tid * 32 + b);
          p++;
        }
      }
    } else {
      uint32_t m = 0;  // bit e: element e is touched
#pragma unroll
      for (int s = 0; s < BL::S; s++) {
#pragma unroll
        for (int v = 0; v < BL::VEC / 4; v++) {
          const uint4 q = t4[((s * NTH + tid) * BL::VEC) / 4 + v];
          const int e = s * BL::VEC + 4 * v;
          m |= (q.x ? 1u : 0u) << e;
          m |= (q.y ? 1u : 0u) << (e + 1);
          m |= (q.z ? 1u : 0u) << (e + 2);
          m |= (q.w ? 1u : 0u) << (e + 3);
        }
      }
      const int c = __popc(m);
      const int inc = wave_scan_incl<int>(c);
      int wb = 0;
      if (lane_id() == 63 && inc) wb = atomicAdd(np, inc);
      int p = readlane<int>(wb, 63) + inc - c;
      while (m) {
        const int e = __ffs(m) - 1;
        m &= m - 1u;
        if (p < lcap2) list2[p] = (uint32_t)(((e / BL::VEC) * NTH + tid) * BL::VEC + e % BL::VEC);
        p++;
      }
    }
    bar();
    const int n = *np;
    if (n <= lcap2) {
      // each listed token processed by one thread; the value replaces the word (+0 stored as -0 so that the word
      // stays nonzero: every consumer folds -0 and +0), and the owners take the values of their nonzero words
      for (int p = tid; p < n; p += NTH) {
        const int loc = (int)list2[p];
        const float v = proc_one(BL::at(B, R, row, lo + loc), tab[loc], R, bias_row);
        if (patches && n <= TCAP) patches[p] = make_uint2((uint32_t)loc, __float_as_uint(v));
        const uint32_t vb = __float_as_uint(v);
        tab[loc] = vb ? vb : 0x80000000u;
      }
      bar();
#pragma unroll
      for (int s = 0; s < BL::S; s++) {
#pragma unroll
        for (int v = 0; v < BL::VEC / 4; v++) {
          const uint4 q = t4[((s * NTH + tid) * BL::VEC) / 4 + v];
          const int e = s * BL::VEC + 4 * v;
          x[e] = q.x ? __uint_as_float(q.x) : x[e];
          x[e + 1] = q.y ? __uint_as_float(q.y) : x[e + 1];
          x[e + 2] = q.z ? __uint_as_float(q.z) : x[e + 2];
          x[e + 3] = q.w ? __uint_as_float(q.w) : x[e + 3];
        }
      }
    } else {  // more than the list holds: each thread processes its own touched tokens in place
#pragma unroll
      for (int s = 0; s < BL::S; s++) {
#pragma unroll
        for (int v = 0; v < BL::VEC / 4; v++) {
          const uint4 q = t4[((s * NTH + tid) * BL::VEC) / 4 + v];
          const int e = s * BL::VEC + 4 * v;
          if (q.x) x[e] = proc_one(x[e], q.x, R, bias_row);
          if (q.y) x[e + 1] = proc_one(x[e + 1], q.y, R, bias_row);
          if (q.z) x[e + 2] = proc_one(x[e + 2], q.z, R, bias_row);
          if (q.w) x[e + 3] = proc_one(x[e + 3], q.w, R, bias_row);
        }
      }
    }
    if (tail) bar();
    return;
  }
  uint32_t tw[EPT];
  int nt = 0;
#pragma unroll
  for (int s = 0; s < BL::S; s++) {
#pragma unroll
    for (int v = 0; v < BL::VEC / 4; v++) {
      const uint4 q = t4[((s * NTH + tid) * BL::VEC) / 4 + v];
      tw[s * BL::VEC + 4 * v] = q.x;
      tw[s * BL::VEC + 4 * v + 1] = q.y;
      tw[s * BL::VEC + 4 * v + 2] = q.z;
      tw[s * BL::VEC + 4 * v + 3] = q.w;
    }
  }
#pragma unroll
  for (int e = 0; e < EPT; e++) nt += tw[e] ? 1 : 0;
  int slot = 0;
  {  // list slots of this thread's touched tokens: one atomic per wave
    const int inc = wave_scan_incl<int>(nt);
    int wb = 0;
    if (lane_id() == 63 && inc) wb = atomicAdd(np, inc);
    slot = readlane<int>(wb, 63) + inc - nt;
  }
  if (lcap2 > 0) {  // list the touched tokens in list2 while the table may still be read
    float* lx = (float*)list2;
    uint32_t* lw = list2 + lcap2;
    uint32_t* lj = list2 + 2 * lcap2;
    int sl = slot;
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      if (tw[e]) {
        if (sl < lcap2) {
          lx[sl] = x[e];
          lw[sl] = tw[e];
          lj[sl] = (uint32_t)BL::local(e);
        }
        sl++;
      }
    }
  }
  bar();  // every table word has been read: the region holds the list from here on
  const int n = *np;
  if (n <= lcap2) {  // process the listed tokens one per thread, hand the values back
    float* lx = (float*)list2;
    const uint32_t* lw = list2 + lcap2;
    const uint32_t* lj = list2 + 2 * lcap2;
    for (int p = tid; p < n; p += NTH) {
      const float v = proc_one(lx[p], lw[p], R, bias_row);
      lx[p] = v;
      if (patches && n <= TCAP) patches[p] = make_uint2(lj[p], __float_as_uint(v));
    }
    bar();
    int sl = slot;
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      if (tw[e]) {
        x[e] = lx[sl];
        sl++;
      }
    }
  } else if (n <= LCAP) {  // compact the touched tokens, process them one per thread, hand the values back
    float* lx = (float*)tab;
    uint32_t* lw = tab + LCAP;
    uint32_t* lj = tab + 2 * LCAP;
    int sl = slot;
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      if (tw[e]) {
        lx[sl] = x[e];
        lw[sl] = tw[e];
        lj[sl] = (uint32_t)BL::local(e);
        sl++;
      }
    }
    bar();
    for (int p = tid; p < n; p += NTH) {
      const float v = proc_one(lx[p], lw[p], R, bias_row);
      lx[p] = v;
      if (patches && n <= TCAP) patches[p] = make_uint2(lj[p], __float_as_uint(v));
    }
    bar();
    sl = slot;
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      if (tw[e]) {
        x[e] = lx[sl];
        sl++;
      }
    }
  } else {  // many touched tokens: in place
#pragma unroll
    for (int e = 0; e < EPT; e++)
      if (tw[e]) x[e] = proc_one(x[e], tw[e], R, bias_row);
  }
  if (tail) bar();
}

}  // namespace qws
