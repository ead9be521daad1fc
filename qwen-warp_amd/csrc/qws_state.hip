// qws device-resident processor state: per-request touched-token tables kept across decode steps.
//
// The reference keeps dense per-request buffers (counts int32[V], flags u8[V], bias f32[V]; ProcBufs,
// engine/src/proc.h:16-35) that proc_begin fills once per request (engine/src/proc.cu:72-103) and proc_note
// updates with the emitted tokens (engine/src/proc.h:52-56, k_note_ids engine/src/proc.cu:53).  Here a slot holds
// only the touched tokens (prompt set and generated counts), split by 8,192-token block, so that a sampling call
// reads its block's entries (a few hundred words) instead of scanning the request's whole history once per block.
//   k_state_begin  (G workgroups): one block's table from the prompt / generated ids, compacted into entries.
//   k_state_note   (B workgroups): the emitted tokens of one slot, deduplicated, each found in its block's entries
//                  and counted, or appended.
//   k_finish       (B workgroups): the bookkeeping of a decode step for each sequence in one launch: output ring,
//                  position, counters, the processor-state note and the PLD history append.
// Layout and entry format: qws_block.h (state_*, SE_*), qws_pld.h (PLD histories).
#include "qws_block.h"
#include "qws_pld.h"

namespace qws {

constexpr int NTS = 512;  // workgroup of both kernels
constexpr int MAXT = 64;  // tokens per slot of one note call (one wave deduplicates them)

__global__ void __launch_bounds__(NTS) k_state_begin(void* mem, int V, int slot, const int* prompt, int n_prompt, const int* gen, int n_gen) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tab[BLK];
  __shared__ uint32_t s_red[NTS / 64];
  const int g = blockIdx.x, tid = threadIdx.x, lo = g * BLK, hi = min(V, lo + BLK);
  for (int i = tid; i < BLK / 4; i += NTS) ((uint4*)s_tab)[i] = make_uint4(0u, 0u, 0u, 0u);
  bar();
  for (int j = tid; j < n_prompt; j += NTS) {
    const int id = prompt[j];
    if (id >= lo && id < hi) atomicOr(&s_tab[id - lo], SE_PROMPT);
  }
  for (int j = tid; j < n_gen; j += NTS) {
    const int id = gen[j];
    if (id >= lo && id < hi) atomicAdd(&s_tab[id - lo], 1u << SE_CNT_SHIFT);
  }
  bar();
  // entries in token order: thread t owns the contiguous table words [t * 16, t * 16 + 16)
  constexpr int PT = BLK / NTS;
  uint32_t w[PT];
#pragma unroll
  for (int v = 0; v < PT / 4; v++) {
    const uint4 q = ((const uint4*)s_tab)[tid * (PT / 4) + v];
    w[4 * v] = q.x;
    w[4 * v + 1] = q.y;
    w[4 * v + 2] = q.z;
    w[4 * v + 3] = q.w;
  }
  uint32_t nz = 0;
#pragma unroll
  for (int k = 0; k < PT; k++) nz += w[k] ? 1u : 0u;
  uint32_t total;
  uint32_t p = block_scan_incl<NTS / 64, uint32_t>(nz, s_red, &total) - nz;
  uint32_t* ent = state_entries(mem, V, slot, g);
#pragma unroll
  for (int k = 0; k < PT; k++)
    if (w[k]) ent[p++] = w[k] | (uint32_t)(tid * PT + k);
  if (tid == 0) state_counts(mem, V, slot)[g] = total;
}

// The tokens toks[0..T) (T <= 64, values outside [0, V) skipped) added to slot `slot`, by the whole workgroup (NTS
// threads): wave 0 deduplicates them (each distinct token once, with its multiplicity) and reads the entry count of
// each one's block before anything is appended; then wave w handles distinct tokens w, w + 8, ...: a search of the
// block's existing entries by all 64 lanes, then a saturating count update of the entry found or an append (a count
// atomic reserves the place).  Distinct tokens never share an entry, and the appended entries lie past the counts
// read first, so no search sees a write of this call.  Called by every thread of the workgroup.
__device__ void state_note_row(void* mem, int V, int slot, const int* toks, int T) {
  __shared__ int s_tok[MAXT], s_mul[MAXT], s_n0[MAXT];
  __shared__ int s_nd;
  const int lane = lane_id(), wave = wave_id();
  uint32_t* cnt = state_counts(mem, V, slot);
  if (wave == 0) {
    const int tok = lane < T ? toks[lane] : -1;
    const bool ok = tok >= 0 && tok < V;
    int mult = 0;
    bool lead = ok;
    for (int u = 0; u < T; u++) {
      const int o = __shfl(tok, u);
      if (ok && o == tok) {
        mult++;
        if (u < lane) lead = false;
      }
    }
    const unsigned long long m = __ballot(lead);
    const int pos = __popcll(m & ((1ull << lane) - 1ull));
    if (lead) {
      s_tok[pos] = tok;
      s_mul[pos] = mult;
      s_n0[pos] = (int)min(cnt[tok / BLK], (uint32_t)BLK);
    }
    if (lane == 0) s_nd = __popcll(m);
  }
  bar();
  const int nd = s_nd;
  for (int d = wave; d < nd; d += NTS / 64) {
    const int tok = s_tok[d], g = tok / BLK;
    const uint32_t local = (uint32_t)(tok - g * BLK);
    const int n0 = s_n0[d];
    uint32_t* ent = state_entries(mem, V, slot, g);
    int found = -1;
    for (int j0 = 0; j0 < n0 && found < 0; j0 += 64 * 4) {
      uint32_t ev[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int j = j0 + k * 64 + lane;
        ev[k] = j < n0 ? ent[j] : 0xFFFFFFFFu;
      }
      int hit = -1;
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (hit < 0 && (ev[k] & SE_LOCAL) == local && ev[k] != 0xFFFFFFFFu) hit = j0 + k * 64 + lane;
      const unsigned long long hm = __ballot(hit >= 0);
      if (hm) found = __shfl(hit, __ffsll((long long)hm) - 1);
    }
    if (lane == 0) {
      if (found >= 0) {
        const uint32_t e = ent[found];
        const uint32_t c = min((e >> SE_CNT_SHIFT) + (uint32_t)s_mul[d], SE_CNT_MAX);
        ent[found] = (e & ((1u << SE_CNT_SHIFT) - 1u)) | (c << SE_CNT_SHIFT);
      } else {
        const uint32_t p = atomicAdd(&cnt[g], 1u);
        if (p < (uint32_t)BLK) ent[p] = local | (min((uint32_t)s_mul[d], SE_CNT_MAX) << SE_CNT_SHIFT);
      }
    }
  }
}

// Slot `slot` expanded to dense per-token arrays (the reference's ProcBufs counts and PF_PROMPT flags, read back by
// smk_engine_read what = 3, engine/include/engine.h:173-176): counts[i] = token i's generated count, flags[i] bit 0 = i is
// in the prompt set.  One workgroup per block: the block's entries scattered into an LDS table, then written out whole.
__global__ void __launch_bounds__(NTS) k_state_read(const void* mem, int V, int slot, int* counts, unsigned char* flags) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tab[BLK];
  const int g = blockIdx.x, tid = threadIdx.x, lo = g * BLK, hi = min(V, lo + BLK);
  for (int i = tid; i < BLK / 4; i += NTS) ((uint4*)s_tab)[i] = make_uint4(0u, 0u, 0u, 0u);
  bar();
  void* m = const_cast<void*>(mem);
  const int n = (int)min(state_counts(m, V, slot)[g], (uint32_t)BLK);
  const uint32_t* ent = state_entries(m, V, slot, g);
  for (int j = tid; j < n; j += NTS) {
    const uint32_t e = ent[j];
    s_tab[e & SE_LOCAL] = e;  // distinct tokens: one entry each
  }
  bar();
  for (int l = tid; l < hi - lo; l += NTS) {
    const uint32_t e = s_tab[l];
    counts[lo + l] = (int)(e >> SE_CNT_SHIFT);
    if (flags) flags[lo + l] = (e & SE_PROMPT) ? 1 : 0;
  }
}

__global__ void __launch_bounds__(NTS) k_state_note(void* mem, int slots, int V, const int* row_slots, const int* tokens, int T) {
  const int b = blockIdx.x;
  const int slot = row_slots[b];
  if (slot < 0 || slot >= slots) return;
  state_note_row(mem, V, slot, tokens + (size_t)b * T, T);
}

// Step bookkeeping of sequence row_seqs[b] (the reference's spec_finish, engine/src/mtp_sample.h:65-92, with
// proc_note, engine/src/proc.h:52-56, and the proposer's append, engine/src/pld.cu:71-76): a = counts[b] tokens
// (or the tokens before the first negative one when counts is null), clamped to [0, T].
// With `rows` (the next call's row array, rows_per_entry rows per entry b), the rows of entry b advance as the
// reference's cycle state does: the Philox counter word 0 by one per cycle (ss[SS_NCYC], engine/src/mtp_sample.h:80)
// and ngen by the a tokens emitted (proc_note, engine/src/proc.h:52-56).
// With `force` (n_force > 0 entries, the reference's SS_FORCE schedule, engine/src/mtp_sample.h:68-70, a rollback test):
// a sequence whose step is its cycles-th keeps a = min(a, f) tokens, f = force[cycles % n_force] when 1 <= f; the
// accepted-length histogram still counts the natural a.
__global__ void __launch_bounds__(NTS) k_finish(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, const int* tokens,
                                               const int* counts, int T, void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs,
                                               int pld_max_len, qws_row* rows, int rows_per_entry, const int* force, int n_force) {
  const int b = blockIdx.x, tid = threadIdx.x, lane = lane_id();
  const int* y = tokens + (size_t)b * T;
  const int t = lane < T ? y[lane] : -1;
  int a;
  if (counts) {
    a = min(max(counts[b], 0), T);
  } else {
    const unsigned long long neg = __ballot(t < 0);
    a = neg ? __ffsll((long long)neg) - 1 : T;
  }
  const int s = row_seqs[b];
  const bool has_seq = s >= 0 && s < nseq;
  const int a_nat = a;
  if (force && n_force > 0 && has_seq) {  // the schedule is indexed by the sequence's cycle count
    const int f = force[seqs[s].cycles % n_force];
    if (f >= 1 && f < a) a = f;
  }
  if (rows && tid < rows_per_entry) {
    qws_row& r = rows[(size_t)b * rows_per_entry + tid];
    r.position += 1u;
    r.ngen += a;
  }
  if (!has_seq) return;
  __syncthreads();  // every read of the sequence's cycle count above comes before its update below
  if (tid < 64) {
    qws_seq& q = seqs[s];
    const int outn = q.outn;
    if (lane < a) rings[(size_t)s * ring_len + (outn + lane) % ring_len] = t;
    if (lane == 0 && a > 0) {
      q.outn = outn + a;
      q.pos += a;
      q.last = y[a - 1];
      q.cycles += 1;
      q.hist[min(a_nat - 1, 7)] += 1;
    }
    if (pld_mem && s < pld_seqs && a > 0) pld_append_wave(pld_mem, pld_max_len, s, t, a);
  }
  if (state_mem && s < state_slots && a > 0) state_note_row(state_mem, V, s, y, a);
}

}  // namespace qws

static int finish_launch(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, int B, const int* tokens, const int* counts, int T,
                         void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs, int pld_max_len, qws_row* rows, int rows_per_entry,
                         void* stream, const int* force = nullptr, int n_force = 0) {
  using namespace qws;
  if (!seqs || nseq < 1 || !rings || ring_len < 1 || !row_seqs || !tokens || B < 0 || T < 1 || T > MAXT) return QWS_ERR_INVALID;
  if (state_mem && (((uintptr_t)state_mem & 255) || state_slots < 1 || V < 8)) return QWS_ERR_INVALID;
  if (state_mem && (V + BLK - 1) / BLK > 64) return QWS_ERR_NOT_SUPPORTED;
  if (pld_mem && (((uintptr_t)pld_mem & 255) || pld_seqs < 1 || pld_max_len < 1)) return QWS_ERR_INVALID;
  if (rows && (rows_per_entry < 1 || rows_per_entry > 64)) return QWS_ERR_INVALID;
  if (n_force < 0 || (n_force > 0 && !force)) return QWS_ERR_INVALID;
  if (B == 0) return QWS_OK;
  hipLaunchKernelGGL(k_finish, dim3(B), dim3(NTS), 0, (hipStream_t)stream, seqs, nseq, rings, ring_len, row_seqs, tokens, counts, T, state_mem,
                     state_slots, V, pld_mem, pld_seqs, pld_max_len, rows, rows ? rows_per_entry : 0, force, n_force);
  return (int)hipGetLastError();
}

extern "C" int qws_finish(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, int B, const int* tokens, const int* counts, int T,
                          void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs, int pld_max_len, void* stream) {
  return finish_launch(seqs, nseq, rings, ring_len, row_seqs, B, tokens, counts, T, state_mem, state_slots, V, pld_mem, pld_seqs, pld_max_len, nullptr, 0,
                       stream);
}

extern "C" int qws_finish_rows(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, int B, const int* tokens, const int* counts, int T,
                               void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs, int pld_max_len, qws_row* rows,
                               int rows_per_entry, void* stream) {
  if (!rows) return QWS_ERR_INVALID;
  return finish_launch(seqs, nseq, rings, ring_len, row_seqs, B, tokens, counts, T, state_mem, state_slots, V, pld_mem, pld_seqs, pld_max_len, rows,
                       rows_per_entry, stream);
}

extern "C" int qws_finish_forced(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, int B, const int* tokens, const int* counts,
                                 int T, void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs, int pld_max_len, qws_row* rows,
                                 int rows_per_entry, const int* force, int n_force, void* stream) {
  return finish_launch(seqs, nseq, rings, ring_len, row_seqs, B, tokens, counts, T, state_mem, state_slots, V, pld_mem, pld_seqs, pld_max_len, rows,
                       rows_per_entry, stream, force, n_force);
}

extern "C" size_t qws_state_bytes(int slots, int V) {
  if (slots < 1 || V < 8 || (V + qws::BLK - 1) / qws::BLK > 64) return 0;
  return (size_t)slots * qws::state_slot_bytes(V);
}

extern "C" int qws_state_begin(void* state_mem, int slots, int V, int slot, const int* prompt, int n_prompt, const int* gen, int n_gen, void* stream) {
  using namespace qws;
  if (!state_mem || ((uintptr_t)state_mem & 255) || slots < 1 || V < 8 || slot < 0 || slot >= slots) return QWS_ERR_INVALID;
  if (n_prompt < 0 || n_gen < 0 || (n_prompt > 0 && !prompt) || (n_gen > 0 && !gen) || n_gen > (int)SE_CNT_MAX) return QWS_ERR_INVALID;
  const int G = (V + BLK - 1) / BLK;
  if (G > 64) return QWS_ERR_NOT_SUPPORTED;
  hipLaunchKernelGGL(k_state_begin, dim3(G), dim3(NTS), 0, (hipStream_t)stream, state_mem, V, slot, prompt, n_prompt, gen, n_gen);
  return (int)hipGetLastError();
}

extern "C" int qws_state_note(void* state_mem, int slots, int V, const int* row_slots, int B, const int* tokens, int T, void* stream) {
  using namespace qws;
  if (!state_mem || ((uintptr_t)state_mem & 255) || slots < 1 || V < 8 || !row_slots || !tokens || B < 0 || T < 1 || T > MAXT)
    return QWS_ERR_INVALID;
  if ((V + BLK - 1) / BLK > 64) return QWS_ERR_NOT_SUPPORTED;
  if (B == 0) return QWS_OK;
  hipLaunchKernelGGL(k_state_note, dim3(B), dim3(NTS), 0, (hipStream_t)stream, state_mem, slots, V, row_slots, tokens, T);
  return (int)hipGetLastError();
}

extern "C" int qws_state_read(const void* state_mem, int slots, int V, int slot, int* counts, unsigned char* flags, void* stream) {
  using namespace qws;
  if (!state_mem || ((uintptr_t)state_mem & 255) || slots < 1 || V < 8 || slot < 0 || slot >= slots || !counts) return QWS_ERR_INVALID;
  const int G = (V + BLK - 1) / BLK;
  if (G > 64) return QWS_ERR_NOT_SUPPORTED;
  hipLaunchKernelGGL(k_state_read, dim3(G), dim3(NTS), 0, (hipStream_t)stream, state_mem, V, slot, counts, flags);
  return (int)hipGetLastError();
}
