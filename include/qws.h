/* qws: MI355X-native sampling stage for qwen-warp's decode loop (C ABI).
 *
 * One shared library, libqws.so (HIP, gfx950).  Every entry point returns an int status: 0 = OK,
 * QWS_ERR_INVALID (= hipErrorInvalidValue = cudaErrorInvalidValue, 1) for rejected arguments,
 * QWS_ERR_NOT_SUPPORTED (801, as cudaErrorNotSupported) for shapes the kernels do not handle, and
 * any other HIP error code unchanged -- the reference's cudaError_t convention
 * (engine/src/mtp.cu:484-498, engine/src/proc.cu:80-82; checked by engine/smk.py:48-50).
 *
 * Device pointers come from the caller (torch tensors' data_ptr()); `stream` is a hipStream_t.
 * The batched entry points (qws_sample, qws_verify) allocate nothing: the caller passes a device
 * workspace of at least the queried size, so they are stream-ordered and capturable.  The test hooks
 * (qws_test_*) take host arrays, allocate their own scratch and synchronise, like the reference's
 * smk_test_* hooks (engine/src/mtp_sample.cu:440-599, engine/src/proc.cu:211-250).
 */
#ifndef QWS_H
#define QWS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWS_OK 0
#define QWS_ERR_INVALID 1
#define QWS_ERR_NOT_SUPPORTED 801

#define QWS_DTYPE_F32 0
#define QWS_DTYPE_BF16 1

#define QWS_MASK_NONE 0
#define QWS_MASK_BANNED 1  /* bit set = token masked (-inf) */
#define QWS_MASK_ALLOWED 2 /* bit clear = token masked: allowed_token_ids as a bitmask */

/* Philox counter word 1 ("stream") values of the reference (engine/src/mtp_sample.h:45). */
#define QWS_ST_ACCEPT 0x1000u
#define QWS_ST_DRAFT 0x2000u
#define QWS_ST_FIRST 0x3000u
#define QWS_ST_DRAW 0x4000u

/* qws_row.test_flags (TEST ONLY; no reference counterpart beyond bit 0) */
#define QWS_TF_BROKEN 1u /* verify: resample from p, not the residual (the reference's SampP.flags bit0 control) */
#define QWS_TF_RESCAN 2u /* take every cut bin's elements from rescans of the blocks, not from the first pass's lists */
#define QWS_TF_STAGED_DRAW 4u /* draw inside the drawn block from a rescan of it even when its kept set lies in its list */
#define QWS_TF_SPLIT_SELECT 8u /* a cut bin gathered, then selected, in separate passes even when all of it is listed */

/* Same layout and meaning as the reference's smk_sampling (engine/include/mtp.h:97-108), so a
 * ctypes Structure built by engine/spec.py:40-46 (make_sampling) binds unchanged.  Used by the
 * host-fed test hook qws_test_dist and by the Python layer to fill qws_row. */
typedef struct qws_sampling {
  float temperature;       /* 0 = greedy */
  int top_k;               /* <= 0: no top-k filter (the reference limits 1..64, see qws_row) */
  float top_p;             /* (0, 1] */
  int draft_sample;        /* reference field; qws_verify takes the draft tokens as input */
  float draft_temperature; /* reference field (unused) */
  int draft_top_k;         /* reference field (unused) */
  float draft_top_p;       /* reference field (unused) */
  int test_flags;          /* TEST ONLY.  bit0: broken verify (resample from p, not the residual) */
  unsigned long long seed;
  float min_p;             /* [0, 1], 0 = off */
} qws_sampling;

/* Same layout and meaning as the reference's smk_procs (engine/include/engine.h:142-154), host arrays. */
typedef struct qws_procs {
  float presence, frequency, repetition; /* 0, 0, 1 = off */
  int min_tokens;
  const int* prompt;
  int n_prompt;
  const int* bias_ids;
  const float* bias_vals;
  int n_bias;
  const int* allowed;
  int n_allowed;
  const int* stop;
  int n_stop;
} qws_procs;

/* One logits row of a batched call (device memory, 128 bytes).  Replaces the reference's per-request
 * device state SampP + ProcP (engine/src/mtp_sample.h:32-42, engine/src/proc.h:16-25): the batch loop
 * passes every row's sampling parameters and token history with each call.
 *   history: hist[hist_off .. hist_off + n_prompt) = prompt ids (repetition penalty only), then
 *            n_gen generated ids (counts for frequency / presence, and the repetition set);
 *   drafts:  drafts[draft_off .. draft_off + n_drafts) count as generated as well (verify row t of
 *            a speculative cycle sees d_1..d_t: engine/src/proc.cu:24); ngen counts them too;
 *   bias:    bias_ids / bias_vals[bias_off .. bias_off + n_bias), distinct ids;
 *   stop:    stop_ids[stop_off .. stop_off + n_stop), masked while min_tokens > ngen + n_drafts;
 *   mask:    masks[mask_row * mask_words ..] interpreted by mask_mode (QWS_MASK_*);
 *   state:   state_slot >= 0: slot of the batch's qws_state arena whose per-request counts and prompt set
 *            (qws_state_begin / qws_state_note) apply to the row as well (its CSR history is then normally
 *            empty: n_prompt = n_gen = 0); -1: none. */
typedef struct qws_row {
  float temperature; /* <= 0: greedy (argmax of the processed logits) */
  int top_k;         /* <= 0: off */
  float top_p;       /* (0, 1]; 1 = off */
  float min_p;       /* [0, 1]; 0 = off */
  double log2_min_p; /* log2(min_p), filled by qws_row_init / the host (ignored when min_p == 0) */
  unsigned long long seed;
  unsigned position; /* Philox counter word 0 */
  unsigned stream;   /* counter word 1 */
  unsigned row_key;  /* counter word 2 */
  int proc_on;       /* 0: no processors (the logits are used as given; NaN -> -inf) */
  float presence, frequency, repetition;
  int min_tokens;
  int ngen; /* tokens generated before this row (excluding the drafts below) */
  int hist_off, n_prompt, n_gen;
  int draft_off, n_drafts;
  int bias_off, n_bias;
  int stop_off, n_stop;
  int mask_mode, mask_row;
  int test_flags;
  int draw_word; /* Philox output word of the row's draw: 0 = x (sampling), 1 = y (the verify rows' residual
                    and bonus draws, engine/src/mtp_sample.cu:250,255) */
  int state_slot; /* slot of batch.state_mem, or -1 */
  int pad_;
} qws_row;

/* A batched sampling call: B rows of logits [B][row_stride] (dtype QWS_DTYPE_*), V tokens per row.
 * Limits: V % 8 == 0, row_stride % 8 == 0 (0 = every row reads row 0), 16-byte aligned logits,
 * n_gen + n_drafts <= 65535 and n_bias <= 2047 per row.  Zero-initialise the struct (memset, or = {0} in C) before
 * filling it field by field: every field is read, `advance` included. */
typedef struct qws_batch {
  const void* logits;
  int dtype;
  int B, V;
  long long row_stride;
  const qws_row* rows; /* device [B] */
  const int* hist;
  const int* drafts;
  const int* bias_ids;
  const float* bias_vals;
  const int* stop_ids;
  const unsigned* masks;
  int mask_words;      /* uint32 words per mask row (>= V / 32) */
  int* out_tokens;     /* device [B] */
  float* out_logits;   /* optional device [B][V]: processed logits (test hook path), else NULL */
  float* out_probs;    /* optional device [B][V]: sampling probabilities, else NULL.  Every entry is written: 0 outside
                          the kept set, 1 at a greedy row's token (the point mass), all 0 for a row without a
                          candidate, so a reused buffer needs no clearing */
  int* out_info;       /* optional device [B]: 0 = resolved from the first pass's records, 1 = the same with rescans of
                          blocks whose listed window missed the cut bin, 2 = greedy */
  void* state_mem;     /* qws_state arena of the rows' state_slot (NULL when no row uses one) */
  int state_slots;     /* slots of that arena */
  int advance;         /* nonzero (qws_sample): each row also takes the step on the device -- its token added to its
                          state slot as qws_state_note would (the reference's proc_note, engine/src/proc.h:52-56), and
                          its ngen and position (Philox counter word 0, the reference's cycle counter ss[SS_NCYC],
                          engine/src/mtp_sample.h:80) incremented in `rows`, which the call then writes.  A row without
                          a candidate (every logit -inf or masked) emits token 0, the greedy token of such a row, and
                          takes the step with it, as qws_finish_rows does with the same output.  Rows of one call must
                          then have distinct state slots, and a row whose penalties count generated tokens must keep
                          them in its state slot (n_prompt = n_gen = 0): a CSR history in `hist` is not extended by
                          the step, so its counts would miss the drawn tokens.  Ignored by qws_verify; qws_draft_pick
                          rejects it (QWS_ERR_INVALID). */
} qws_batch;

/* Workspace bytes for qws_sample with B rows of V tokens. */
size_t qws_sample_ws_bytes(int B, int V);
/* Processors + greedy / temperature, min_p, top-k, top-p and a Philox draw for every row.
 * Replaces the sampling path of the reference's head tail and sk_topk + sample
 * (engine/src/engine.cu:31-49 proc_logits; engine/src/mtp_sample.cu:397-411 sk_topk;
 *  engine/src/mtp_sample.cu:298-311 k_first_pick; engine/include/mtp.h:89-113). */
int qws_sample(const qws_batch* b, void* ws, size_t ws_bytes, void* stream);

/* qws_sample without a workspace argument, for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.  The workspace is a
 * library-owned device array of QWS_NOALLOC_SCRATCH_BYTES per GPU (16 MiB, held until the process ends; its device
 * address is taken once per device on the first call there).  Calls whose qws_sample_ws_bytes(B, V) exceeds it
 * return QWS_ERR_NOT_SUPPORTED (at V = 248,320: at most 15 rows).  Allocates nothing.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (concurrent streams, or threads) race and must be serialised by
 * the caller; consecutive calls on one stream are safe (nothing in the array needs clearing between calls). */
#define QWS_NOALLOC_SCRATCH_BYTES (16u << 20)
int qws_sample_noalloc(const qws_batch* b, void* stream);

/* A speculative verify call (the reference's accept_core + residual + bonus, engine/src/mtp_sample.cu:227-258,
 * k_accept_s :266-278, over the Dist rows of sk_topk :397-411): B sequences, each with K draft tokens
 * d_1..d_K proposed by a drafter over a reduced vocabulary of Vd ids and K + 1 target logits rows.
 *   target: B * (K + 1) rows; row b * (K + 1) + t is target row t of sequence b, with d_1..d_t among its
 *           drafts (the processors count them as generated, engine/src/proc.cu:24), stream QWS_ST_ACCEPT + t
 *           and draw_word 1 (the reference's rng(ctr, ACCEPT + t): .x for the test, .y for the residual or
 *           bonus draw).  target.out_tokens is not used (the rows' own draws go to the workspace).
 *   draft_tokens [B][K]: target ids; draft_probs [B][K][Vd]: q of draft step t over the reduced vocabulary;
 *   inv_map [V]: reduced index of each target id or -1 (qws_verify_map), 16-byte aligned.
 * Draft t is accepted iff u * floor(q(d_t) * S2) < w(d_t) * 2^24 (u = 24-bit .x, w / S2 the exact fixed-point
 * p of row t); the first rejected draft is replaced by a draw from max(0, p - q) over p's support (from p when
 * that is empty, or when the row has test_flags & QWS_TF_BROKEN); with all K accepted the bonus is drawn from
 * row K.  Out: out_tokens [B][K + 1] (emitted tokens, -1 past out_n[b]) and out_n [B] = accepted drafts + 1. */
typedef struct qws_verify_batch {
  qws_batch target;
  int B, K, Vd; /* 1 <= K <= 15 */
  const int* draft_tokens;
  const float* draft_probs;
  const int* inv_map;
  int* out_tokens;
  int* out_n;
  /* Optional device [B] (NULL: every draft is a chain draft).  Drafts t >= n_chain[b] of sequence b are delta
   * proposals -- the prompt-lookup tail tokens of an "MTP chain + PLD tail" cycle (engine/include/mtp.h:66-68,
   * k_delta_q engine/src/mtp_sample.cu:286-296): q = 1 at the draft, so it is accepted with probability p(d) and a
   * rejection draws from p without d; their draft_probs rows are not read. */
  const int* n_chain;
} qws_verify_batch;

size_t qws_verify_ws_bytes(int B, int K, int V);
/* The drafter's picks (the drafter's sk_topk with its own parameters, engine/src/mtp_sample.cu:122-183 with sel = 1,
 * then k_draft_pick :280-284 and the idmap gather of k_topk2 :175; engine/src/mtp.cu:112-119): b holds B rows of
 * draft-head logits over the drafter's reduced vocabulary (b->V = Vd), each row built by
 * qws_row_init_pick(QWS_PICK_DRAFT, j).  Runs qws_sample on them (b->out_tokens = the drawn reduced index,
 * b->out_probs when given = q over the reduced vocabulary, the draft_probs row qws_verify takes) and writes
 * out_ids[b] = idmap[reduced index], the target id (-1 when idmap has no entry).  ws: qws_sample_ws_bytes(B, Vd). */
int qws_draft_pick(const qws_batch* b, const int* idmap, int* out_ids, void* ws, size_t ws_bytes, void* stream);
/* Verifies vb->B sequences of K drafts against their K + 1 target rows each (vb->target, B * (K + 1) rows; row t of a
 * sequence counts d_1..d_t as generated tokens).  vb->target.out_probs / out_logits, when given ([B * (K + 1)][V]):
 * every verify row's sampling distribution (as qws_sample writes it) / processed logits -- the reference's read-back
 * of the processed verify-row distributions (smk_spec_read what = 2, engine/include/mtp.h:57-59).  target.out_tokens
 * is not used. */
int qws_verify(const qws_verify_batch* vb, void* ws, size_t ws_bytes, void* stream);
/* inv_map [V] <- -1, then inv_map[idmap[j]] = j for j < Vd (ids outside [0, V) skipped; a repeated id keeps its
 * largest j).  Build once per draft table: the reference gathers the drafter's reduced ids through the same
 * table (engine/src/mtp_sample.cu:175, idmap in k_topk2). */
int qws_verify_map(const int* idmap, int Vd, int V, int* inv_map, void* stream);

/* Device-resident per-request processor state (the reference's ProcBufs counts + PF_PROMPT flags, kept across
 * decode steps: proc_begin engine/src/proc.cu:72-103, proc_note engine/src/proc.h:52-56 / k_note_ids
 * engine/src/proc.cu:53).  An arena of `slots` slots, each the touched-token table of one request split by
 * 8,192-token block: per block the tokens that occur in the prompt or among the generated ones, with their
 * generated count, so that a sampling call reads only its block's entries instead of the whole history.  The
 * caller allocates qws_state_bytes(slots, V) bytes of device memory (256-byte aligned) and names a slot per row
 * (qws_row.state_slot, qws_batch.state_mem / state_slots).  Counts saturate at 65,471 per token.
 *   qws_state_begin: slot <- prompt ids (prompt set) and gen ids (counts), device arrays; replaces the slot.
 *                    Ids outside [0, V) are skipped (the Python layer rejects them first, as proc_begin's ids_ok,
 *                    engine/src/proc.cu:55-59); n_gen <= 65,471.
 *   qws_state_note:  for b < B with row_slots[b] in [0, slots) (device array), adds tokens[b * T + t], t < T <= 64
 *                    (device; values outside [0, V) skipped, e.g. the -1 after a verify call's emitted tokens),
 *                    to that slot's counts.  The entries of one call must name distinct slots.
 * Both are stream-ordered and allocate nothing. */
size_t qws_state_bytes(int slots, int V);
int qws_state_begin(void* state_mem, int slots, int V, int slot, const int* prompt, int n_prompt, const int* gen, int n_gen, void* stream);
int qws_state_note(void* state_mem, int slots, int V, const int* row_slots, int B, const int* tokens, int T, void* stream);
/* Read-back of one slot (the reference's smk_engine_read what = 3, the request's generated-token counts int[V],
 * engine/include/engine.h:173-176): counts[i] = token i's generated count (device int32 [V]); flags (optional, device
 * uint8 [V]): bit 0 = token i is in the prompt set.  Stream-ordered; allocates nothing.  The rest of the reference's
 * per-request ProcP (what = 4) is the caller's qws_row, which the caller owns on the device. */
int qws_state_read(const void* state_mem, int slots, int V, int slot, int* counts, unsigned char* flags, void* stream);

/* Per-sequence decode-step bookkeeping on the device (the reference's spec_finish, engine/src/mtp_sample.h:65-92,
 * which the cycle's last kernel runs after the accept decision): with a = tokens emitted this step, a sequence's
 * output ring receives them, pos advances by a, last = the last of them, cycles += 1, hist[min(a - 1, 7)] += 1. */
typedef struct qws_seq {
  int pos;     /* position of the next token */
  int last;    /* the last emitted token (the next step's anchor) */
  int outn;    /* tokens written to the output ring (ring index = outn % ring_len) */
  int cycles;  /* steps finished with at least one token */
  int hist[8]; /* steps by emitted tokens - 1 (accepted drafts; 7 = 7 or more) */
} qws_seq;
/* One launch for B rows: row b belongs to sequence row_seqs[b] (device [B]; out-of-range skipped, distinct per call);
 * its tokens are tokens[b * T ..], T <= 64, a = counts[b] (device [B], e.g. qws_verify's out_n) or, with counts
 * NULL, the tokens before the first negative one.  seqs: device [nseq]; rings: device [nseq][ring_len].  Optional
 * (NULL: skipped): the processor-state arena (qws_state_*, slot = sequence index) is noted with the tokens, and the
 * PLD arena (qws_pld_*, sequence index) appends them -- the reference's proc_note (engine/src/proc.h:52-56) and
 * smk_pld_append, in the same launch. */
int qws_finish(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, int B, const int* tokens, const int* counts, int T,
               void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs, int pld_max_len, void* stream);

/* qws_finish that also advances the next step's rows on the device, so that a decode step -- qws_sample or qws_verify,
 * then this -- needs nothing from the host and replays from a captured graph (the reference's cycle graphs advance
 * their counter ss[SS_NCYC] in spec_finish and ngen in proc_note: engine/src/mtp_sample.h:80, engine/src/proc.h:52-56).
 * rows: the device qws_row array the next call reads, rows_per_entry (1..64) rows per entry b -- one for a sampling
 * row, the K + 1 target rows of a verify sequence.  For every b < B (with or without a sequence), with a = the tokens
 * emitted for b: position += 1 (counter word 0 counts cycles, as ss[SS_NCYC]) and ngen += a.  A row's penalties then
 * come from the processor state the same launch notes (state_slot rows), its drafts from the drafts array the drafter
 * writes in place. */
int qws_finish_rows(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, int B, const int* tokens, const int* counts, int T,
                    void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs, int pld_max_len, qws_row* rows, int rows_per_entry,
                    void* stream);

/* qws_finish_rows with the reference's forced-acceptance schedule (smk_spec_set_force, engine/include/mtp.h:49-50; the
 * SS_FORCE rule of spec_finish, engine/src/mtp_sample.h:68-70), a rollback test: a sequence's step keeps
 * a = min(a, f) of its emitted tokens, f = force[cycles % n_force] (force: device [n_force]; f < 1 leaves a as is), and
 * the ring, position, last token, processor-state note, PLD append and the rows' ngen take that a; the accepted-length
 * histogram counts the natural a.  rows may be NULL (then as qws_finish).  n_force = 0: no schedule. */
int qws_finish_forced(qws_seq* seqs, int nseq, int* rings, int ring_len, const int* row_seqs, int B, const int* tokens, const int* counts, int T,
                      void* state_mem, int state_slots, int V, void* pld_mem, int pld_seqs, int pld_max_len, qws_row* rows, int rows_per_entry,
                      const int* force, int n_force, void* stream);

/* Prompt-lookup (PLD) tail proposer with its history on the device: the reference's host proposer
 * (engine/include/pld.h:13-39, engine/src/pld.cu) with the committed tokens kept in HBM, so that a cycle's tail
 * proposal follows the verify call that produced them without a device-to-host round trip
 * (engine/src/mtp.cu:430-437 waits on a mailbox for them).  qws_pld_cfg has smk_pld_cfg's layout and meaning
 * (clamped as smk_pld_create, engine/src/pld.cu:54-62; longest rows examine at most 4,096 candidates).  An arena
 * of `seqs` sequences of at most `max_len` tokens, qws_pld_bytes(seqs, max_len) bytes of device memory (256-byte
 * aligned); all token arrays are device arrays.
 *   qws_pld_reset:   sequence seq <- ctx[0..n) (smk_pld_reset; the last token is the anchor).
 *   qws_pld_append:  for b < B with row_seqs[b] in [0, seqs): appends toks[b * T + t], t < T <= 64, up to the first
 *                    negative value (smk_pld_append).  Tokens beyond max_len mark the sequence overflowed: its
 *                    proposals are empty until the next reset.
 *   qws_pld_propose: for b < B: the tail proposed for sequence row_seqs[b] after drafts[b * nd .. + nd)
 *                    (smk_pld_propose_ex with max_tail <= 8 and min_len per call): out[b * 8 ..] (the tail, -1
 *                    after it), out_n[b] (its length), out_l[b] (the agreement length, 0 without a candidate). */
typedef struct qws_pld_cfg {
  int n, min_len, max_tail, cap, back, longest;
} qws_pld_cfg;
void qws_pld_default_cfg(qws_pld_cfg* c);
size_t qws_pld_bytes(int seqs, int max_len);
int qws_pld_reset(void* mem, int seqs, int max_len, int seq, const int* ctx, int n, void* stream);
int qws_pld_append(void* mem, int seqs, int max_len, const int* row_seqs, int B, const int* toks, int T, void* stream);
int qws_pld_propose(void* mem, int seqs, int max_len, const qws_pld_cfg* cfg, const int* row_seqs, int B, const int* drafts, int nd, int max_tail,
                    int min_len, int* out, int* out_n, int* out_l, void* stream);

/* Candidate select + exact rescore over a quantised head's approximate logits (the reference's
 * smk_headq_select_rescore_ids, engine/include/head_q.h:29-38, engine/src/head_q.cu:124-302).  logits [T][N] fp32
 * (16-byte aligned, N % 4 == 0, N <= 262,144, T <= 16) hold the approximate logits; w_bf16 [rows][K] the BF16 head,
 * x [T][K] bf16 the hidden states (K % 8 == 0, both 16-byte aligned); 1 <= R <= 64.  Per row t: the R best
 * candidates by approximate logit (larger value, then lower index; NaN never), their logits recomputed from the
 * BF16 head (fp32 accumulation of exact bf16 products, in this library's order) and written over logits[t][cand],
 * and the argmax over them (lowest token id on ties) -> out_tok[t], out_val[t] (optional).  ids (optional, device
 * [N], ascending): logits row i is token ids[i] (a sub-vocabulary); candidates and out_tok are then token ids.
 * ws: qws_head_ws_bytes() bytes, 256-byte aligned (no zeroing needed).  The candidates (rank order, -1 past the
 * last) and their exact logits stay in ws: qws_head_ws_cand / qws_head_ws_exact, [16][64] each. */
size_t qws_head_ws_bytes(void);
int qws_head_select_rescore(float* logits, const void* w_bf16, const void* x, int N, int K, int T, int R, int* out_tok, float* out_val, void* ws,
                            void* stream, const int* ids);
const int* qws_head_ws_cand(const void* ws);
const float* qws_head_ws_exact(const void* ws);

/* Argmax over fp32 logits [T][N] -> out_tok[t] (lowest index on ties, NaN never wins) and optional
 * out_val[t].  Same signature and contract as the reference's smk_argmax
 * (engine/include/engine.h:68-71, engine/src/misc.cu:133-137); ws of qws_argmax_ws_bytes() bytes. */
size_t qws_argmax_ws_bytes(void);
int qws_argmax(const float* logits, int T, int N, int* out_tok, float* out_val, void* ws, void* stream);

/* The parameter checks of the reference's smk_spec_set_sampling / valid() (engine/src/mtp_sample.cu:389-392,
 * engine/src/mtp.cu:484-498) and proc_begin (engine/src/proc.cu:78-82) on the reference structs (either may be NULL):
 *   sampling: temperature finite and >= 0 (0 = greedy), top_p in (0, 1], min_p in [0, 1], draft_top_k >= 0,
 *             draft_temperature finite and >= 0, draft_top_p in [0, 1];
 *   procs (only when a processor is active, as proc_begin): repetition > 0, min_tokens >= 0, counts >= 0 with an array
 *             when nonzero, bias_vals given when n_bias > 0, every prompt / bias / allowed / stop id in [0, V) (V <= 0:
 *             ranges not checked), presence, frequency and bias values finite, n_bias <= 65,536.
 * Returns QWS_OK, QWS_ERR_INVALID, or QWS_ERR_NOT_SUPPORTED for 2,047 < n_bias <= 65,536 (this library's per-row
 * limit).  Deliberate difference: top_k is not limited to 1..64 (top_k <= 0 turns top-k off; any k is exact). */
int qws_row_check(const qws_sampling* s, const qws_procs* p, int V);

/* Fills a qws_row from the reference structs (sampling params; processors gating as proc_begin,
 * engine/src/proc.cu:149) and computes log2_min_p; CSR offsets / counts are left to the caller.  Runs
 * qws_row_check(s, p, 0) first and returns its status; a rejected row is left greedy with no processors. */
int qws_row_init(qws_row* r, const qws_sampling* s, const qws_procs* p);

/* The row of one pick of a speculative cycle, from the reference structs (make_sampp, engine/src/mtp_sample.cu:375-387;
 * the picks k_first_pick :298-311, k_draft_pick :280-284, accept_core :227-258, k_draw_n :314-325):
 *   QWS_PICK_FIRST  the cycle's first token from the target logits: target parameters and processors, stream
 *                   QWS_ST_FIRST, word x; test_flags bit1 keeps the engine's argmax (the row is greedy);
 *   QWS_PICK_DRAFT  draft j (j >= 1) from the drafter's logits over its reduced vocabulary: temperature =
 *                   draft_temperature (else temperature), top_k = draft_sample ? (draft_top_k, else top_k) : 1 (q = the
 *                   point mass at the argmax), top_p = draft_top_p (else top_p), no min_p and no processors (the
 *                   target's only), stream QWS_ST_DRAFT + j, word x;
 *   QWS_PICK_VERIFY target row t = j of a verify call: target parameters and processors, stream QWS_ST_ACCEPT + j, word y;
 *   QWS_PICK_DRAW   the test draws: stream QWS_ST_DRAW, word x.
 * Counter word 0 (position), row_key and CSR offsets are left to the caller (0).  Returns qws_row_init's status, or
 * QWS_ERR_INVALID for an unknown kind, a draft j outside 1..4095 or a verify j outside 0..4095. */
#define QWS_PICK_FIRST 0
#define QWS_PICK_DRAFT 1
#define QWS_PICK_VERIFY 2
#define QWS_PICK_DRAW 3
int qws_row_init_pick(qws_row* r, const qws_sampling* s, const qws_procs* p, int kind, int j);

/* sizeof(qws_sampling), sizeof(qws_procs), sizeof(qws_row), sizeof(qws_batch) -> out[4]: lets a binding
 * (ctypes, cgo) check its struct layouts against the library's (no reference counterpart). */
void qws_abi_sizes(size_t* out4);

/* Profiling only (no reference counterpart; the reference's timing hook is smk_spec_launch which=4/5,
 * engine/include/mtp.h:53-56): qws_timing(1) makes qws_sample record HIP events around its two kernels
 * (up to 4096 calls; callers on several threads serialise while it is on); qws_timing_read synchronises them and returns the summed
 * milliseconds of the scan kernel and of the resolver kernel and the number of calls, then clears them. */
int qws_timing(int enable);
int qws_timing_read(float* ms_scan, float* ms_resolve, int* launches);
/* The same for qws_verify's own two kernels (the reference times its verify-row sampling with smk_spec_launch which = 4):
 * the summed milliseconds of the accept / residual-mass kernel and of the residual-draw kernel, and the number of calls
 * (qws_verify's first two kernels, the sampling of its target rows, are counted by qws_timing_read). */
int qws_timing_read_verify(float* ms_accept, float* ms_draw, int* launches);

/* ---------------------------------------------------------------------------------------- test hooks */
/* Philox4x32-10 of counter c[4], key k[2] -> out[4], computed on the GPU (engine/src/mtp_sample.cu:440-453). */
int qws_test_philox(const unsigned* c, const unsigned* k, unsigned* out);
/* Processed logits of host logits [T][N] with the reference's procs and history (gen[n_gen]) and the
 * draft tokens of rows 1..T-1 (engine/include/engine.h:156-158 smk_test_proc_logits). */
int qws_test_proc_logits(const qws_procs* p, int T, int N, const int* gen, int n_gen, const int* drafts,
                         const float* logits, float* out);
/* Processed distributions of host logits [R][N] (fp32): dense probabilities out_p[R][N] and the
 * token drawn with (position, stream) = (ctr, QWS_ST_DRAW) into out_tok[R]
 * (engine/src/mtp_sample.cu:467-487 smk_test_dist, dense instead of <= 64 entries). */
int qws_test_dist(const float* logits, int R, int N, const qws_sampling* cfg, unsigned ctr, float* out_p, int* out_tok);

#ifdef __cplusplus
}
#endif
#endif /* QWS_H */
