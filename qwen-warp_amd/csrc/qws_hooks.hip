// qws: argmax drop-in, row initialisation and the host-fed test hooks.
#include <math.h>
#include <string.h>

#include <vector>

#include "qws_device.h"

namespace qws {
// ---------------------------------------------------------------------------------------------- argmax
// Two launches: per-chunk best (value desc, index asc) -> partial[T][G], then one workgroup per row.
// Same contract as engine/src/misc.cu:50-111 (k_argmax): lowest index on ties, NaN never wins.
constexpr int AM_CHUNK = 4096;
constexpr int AM_GMAX = 1024;
__global__ void __launch_bounds__(256) k_am_part(const float* __restrict__ logits, int N, int G, uint64_t* __restrict__ part) {
  const int row = blockIdx.x / G, g = blockIdx.x % G;
  const int lo = g * AM_CHUNK, hi = min(N, lo + AM_CHUNK);
  const float4* r4 = (const float4*)(logits + (size_t)row * N);
  uint64_t best = 0;
  for (int i = lo / 4 + threadIdx.x; i < hi / 4; i += 256) {
    const float4 v = r4[i];
    const float xs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float x = xs[j] != xs[j] ? -INFINITY : xs[j];
      const uint64_t c = comp(okey(x), (uint32_t)(4 * i + j));
      best = c > best ? c : best;
    }
  }
  best = wave_max_u64(best);
  __shared__ uint64_t red[4];
  if (lane_id() == 0) red[wave_id()] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = red[0];
    for (int i = 1; i < 4; i++) b = red[i] > b ? red[i] : b;
    part[(size_t)row * AM_GMAX + g] = b;
  }
}
__global__ void __launch_bounds__(256) k_am_row(const uint64_t* __restrict__ part, int G, int* out_tok, float* out_val) {
  const int row = blockIdx.x;
  uint64_t best = 0;
  for (int g = threadIdx.x; g < G; g += 256) {
    const uint64_t c = part[(size_t)row * AM_GMAX + g];
    best = c > best ? c : best;
  }
  best = wave_max_u64(best);
  __shared__ uint64_t red[4];
  if (lane_id() == 0) red[wave_id()] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = red[0];
    for (int i = 1; i < 4; i++) b = red[i] > b ? red[i] : b;
    out_tok[row] = (int)(0xFFFFFFFFu - (uint32_t)b);
    if (out_val) out_val[row] = okey_val((uint32_t)(b >> 32));
  }
}

__global__ void k_philox_test(const unsigned* c, const unsigned* k, unsigned* out) {
  uint32_t v[4] = {c[0], c[1], c[2], c[3]};
  philox(v, k[0], k[1]);
  for (int i = 0; i < 4; i++) out[i] = v[i];
}
}  // namespace qws

using namespace qws;

extern "C" size_t qws_argmax_ws_bytes(void) { return (size_t)16 * AM_GMAX * 8; }

extern "C" int qws_argmax(const float* logits, int T, int N, int* out_tok, float* out_val, void* ws, void* stream) {
  if (!logits || !out_tok || !ws || (N & 3) || N < 4 || T < 1 || T > 16 || ((uintptr_t)logits & 15)) return QWS_ERR_INVALID;
  const int G = (N + AM_CHUNK - 1) / AM_CHUNK;
  if (G > AM_GMAX) return QWS_ERR_NOT_SUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_am_part, dim3(T * G), dim3(256), 0, st, logits, N, G, (uint64_t*)ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(k_am_row, dim3(T), dim3(256), 0, st, (const uint64_t*)ws, G, out_tok, out_val);
  return (int)hipGetLastError();
}

static_assert(sizeof(qws_row) == 128, "qws_row layout");
extern "C" void qws_abi_sizes(size_t* out4) {
  out4[0] = sizeof(qws_sampling);
  out4[1] = sizeof(qws_procs);
  out4[2] = sizeof(qws_row);
  out4[3] = sizeof(qws_batch);
}

namespace {
// ids_ok of engine/src/proc.cu:55-59: a count >= 0, an array when it is nonzero, every id in [0, V) (V <= 0: the
// range is not checked, for callers that do not know the vocabulary yet)
bool ids_in(const int* ids, int n, int V) {
  if (n < 0 || (n && !ids)) return false;
  if (V > 0)
    for (int i = 0; i < n; i++)
      if (ids[i] < 0 || ids[i] >= V) return false;
  return true;
}
}  // namespace

// The parameter checks of smk_spec_set_sampling / valid() (engine/src/mtp_sample.cu:389-392, engine/src/mtp.cu:484-498)
// and proc_begin (engine/src/proc.cu:78-82), on the reference structs.  Deliberate differences: temperature 0 is greedy
// (the reference's set_sampling takes it as greedy before valid() too); top_k is not limited to 1..64 (here top_k <= 0
// turns top-k off and any k is exact over the whole vocabulary); presence, frequency and bias values must be finite
// (the reference does not check them; a NaN there would reach the weights); more than 2,047 bias entries is
// QWS_ERR_NOT_SUPPORTED (the per-row limit of this library's block tables), more than 65,536 invalid as in the reference.
extern "C" int qws_row_check(const qws_sampling* s, const qws_procs* p, int V) {
  if (s) {
    const bool ok = s->temperature >= 0.0f && s->temperature < INFINITY && s->top_p > 0.0f && s->top_p <= 1.0f && s->draft_top_k >= 0 &&
                    s->draft_temperature >= 0.0f && s->draft_temperature < INFINITY && s->draft_top_p >= 0.0f && s->draft_top_p <= 1.0f &&
                    s->min_p >= 0.0f && s->min_p <= 1.0f;
    if (!ok) return QWS_ERR_INVALID;
  }
  if (p && (p->presence != 0.0f || p->frequency != 0.0f || p->repetition != 1.0f || p->min_tokens > 0 || p->n_bias > 0 || p->n_allowed > 0)) {
    if (!ids_in(p->prompt, p->n_prompt, V) || !ids_in(p->bias_ids, p->n_bias, V) || !ids_in(p->allowed, p->n_allowed, V) ||
        !ids_in(p->stop, p->n_stop, V) || (p->n_bias && !p->bias_vals) || !(p->repetition > 0.0f) || p->min_tokens < 0 || p->n_bias > 65536)
      return QWS_ERR_INVALID;
    if (!(fabsf(p->presence) < INFINITY) || !(fabsf(p->frequency) < INFINITY)) return QWS_ERR_INVALID;
    for (int i = 0; i < p->n_bias; i++)
      if (!(fabsf(p->bias_vals[i]) < INFINITY)) return QWS_ERR_INVALID;
    if (p->n_bias > 2047) return QWS_ERR_NOT_SUPPORTED;
  }
  return QWS_OK;
}

extern "C" int qws_row_init(qws_row* r, const qws_sampling* s, const qws_procs* p) {
  if (!r) return QWS_ERR_INVALID;
  memset(r, 0, sizeof(*r));
  r->repetition = 1.0f;
  r->top_p = 1.0f;
  r->state_slot = -1;
  r->stream = QWS_ST_FIRST;
  const int e = qws_row_check(s, p, 0);
  if (e) return e;  // the row stays greedy with no processors
  r->temperature = s ? s->temperature : 0.0f;
  r->top_k = s ? s->top_k : 0;
  r->top_p = s ? s->top_p : 1.0f;
  r->min_p = s ? s->min_p : 0.0f;
  r->log2_min_p = r->min_p > 0.0f ? log2((double)r->min_p) : 0.0;
  r->seed = s ? s->seed : 0ull;
  r->test_flags = s ? (s->test_flags & QWS_TF_BROKEN) : 0;  // the sampling config's bit0 (bit1 is a first-pick rule)
  if (p) {  // engine/src/proc.cu:149: any elementwise processor active
    r->presence = p->presence;
    r->frequency = p->frequency;
    r->repetition = p->repetition;
    r->min_tokens = p->min_tokens;
    r->proc_on = p->presence != 0.0f || p->frequency != 0.0f || p->repetition != 1.0f || p->min_tokens > 0 || p->n_bias > 0 || p->n_allowed > 0;
  }
  return QWS_OK;
}

extern "C" int qws_row_init_pick(qws_row* r, const qws_sampling* s, const qws_procs* p, int kind, int j) {
  if (kind < QWS_PICK_FIRST || kind > QWS_PICK_DRAW || (kind == QWS_PICK_DRAFT && (j < 1 || j > 0xFFF)) || (kind == QWS_PICK_VERIFY && (j < 0 || j > 0xFFF))) {
    if (r) (void)qws_row_init(r, nullptr, nullptr);
    return QWS_ERR_INVALID;
  }
  const int e = qws_row_init(r, s, p);
  if (e) return e;
  switch (kind) {
    case QWS_PICK_DRAFT: {  // make_sampp's draft parameters; the drafter's rows have neither min_p nor processors
      const float t = s ? s->temperature : 0.0f;
      r->temperature = (s && s->draft_temperature > 0.0f) ? s->draft_temperature : t;
      r->top_k = (s && s->draft_sample) ? (s->draft_top_k > 0 ? s->draft_top_k : s->top_k) : 1;
      r->top_p = (s && s->draft_top_p > 0.0f) ? s->draft_top_p : (s ? s->top_p : 1.0f);
      r->min_p = 0.0f;
      r->log2_min_p = 0.0;
      r->proc_on = 0;
      r->presence = r->frequency = 0.0f;
      r->repetition = 1.0f;
      r->min_tokens = 0;
      r->stream = QWS_ST_DRAFT + (unsigned)j;
      r->draw_word = 0;
      break;
    }
    case QWS_PICK_VERIFY:
      r->stream = QWS_ST_ACCEPT + (unsigned)j;
      r->draw_word = 1;
      break;
    case QWS_PICK_DRAW:
      r->stream = QWS_ST_DRAW;
      r->draw_word = 0;
      break;
    default:  // QWS_PICK_FIRST; test_flags bit1 keeps the engine's argmax as the first token (k_first_pick)
      r->stream = QWS_ST_FIRST;
      r->draw_word = 0;
      if (s && (s->test_flags & 2)) r->temperature = 0.0f;
      break;
  }
  return QWS_OK;
}

// ---------------------------------------------------------------------------------------------- test hooks
namespace {
struct DevBufs {  // device scratch of one host-fed call, freed on scope exit
  std::vector<void*> ptrs;
  hipError_t err = hipSuccess;
  template <typename T>
  T* alloc(size_t n) {
    void* p = nullptr;
    if (err == hipSuccess) err = hipMalloc(&p, n ? n : 16);
    if (err == hipSuccess) ptrs.push_back(p);
    return (T*)p;
  }
  template <typename T>
  T* up(const T* h, size_t n) {
    T* d = alloc<T>(n * sizeof(T));
    if (err == hipSuccess && n) err = hipMemcpy(d, h, n * sizeof(T), hipMemcpyHostToDevice);
    return d;
  }
  ~DevBufs() {
    for (void* p : ptrs) (void)hipFree(p);
  }
};
bool ids_ok(const int* ids, int n, int V) {
  if (n < 0 || (n && !ids)) return false;
  for (int i = 0; i < n; i++)
    if (ids[i] < 0 || ids[i] >= V) return false;
  return true;
}
}  // namespace

extern "C" int qws_test_philox(const unsigned* c, const unsigned* k, unsigned* out) {
  if (!c || !k || !out) return QWS_ERR_INVALID;
  DevBufs d;
  unsigned* dc = d.up(c, 4);
  unsigned* dk = d.up(k, 2);
  unsigned* dout = d.alloc<unsigned>(16);
  if (d.err != hipSuccess) return (int)d.err;
  hipLaunchKernelGGL(k_philox_test, dim3(1), dim3(1), 0, 0, dc, dk, dout);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpy(out, dout, 16, hipMemcpyDeviceToHost);
  return (int)e;
}

// engine/src/proc.cu:214-229 (smk_test_proc_logits): T verify rows, row t sees drafts[0..t-1] as generated.
extern "C" int qws_test_proc_logits(const qws_procs* p, int T, int N, const int* gen, int n_gen, const int* drafts, const float* logits, float* out) {
  if (!p || T < 1 || N < 8 || (N & 7) || !logits || !out || n_gen < 0 || (n_gen && !gen)) return QWS_ERR_INVALID;
  if (!ids_ok(p->prompt, p->n_prompt, N) || !ids_ok(p->bias_ids, p->n_bias, N) || !ids_ok(p->allowed, p->n_allowed, N) ||
      !ids_ok(p->stop, p->n_stop, N) || !ids_ok(gen, n_gen, N) || (p->n_bias && !p->bias_vals) || !(p->repetition > 0.0f) ||
      p->min_tokens < 0 || p->n_bias > 2047 || n_gen + T > 65535 || (T > 1 && !ids_ok(drafts, T - 1, N)))
    return QWS_ERR_INVALID;
  qws_row r0;
  const int e0 = qws_row_init(&r0, nullptr, p);
  if (e0) return e0;
  std::vector<int> hist;
  hist.insert(hist.end(), p->prompt, p->prompt + p->n_prompt);
  hist.insert(hist.end(), gen, gen + n_gen);
  const int W = (N + 31) / 32;
  std::vector<unsigned> mask;
  if (p->n_allowed > 0) {
    mask.assign(W, 0u);
    for (int i = 0; i < p->n_allowed; i++) mask[p->allowed[i] >> 5] |= 1u << (p->allowed[i] & 31);
  }
  std::vector<qws_row> rows(T, r0);
  for (int t = 0; t < T; t++) {
    qws_row& r = rows[t];
    r.temperature = 0.0f;
    r.hist_off = 0;
    r.n_prompt = p->n_prompt;
    r.n_gen = n_gen;
    r.ngen = n_gen;
    r.draft_off = 0;
    r.n_drafts = t;
    r.bias_off = 0;
    r.n_bias = p->n_bias;
    r.stop_off = 0;
    r.n_stop = p->n_stop;
    r.mask_mode = p->n_allowed > 0 ? QWS_MASK_ALLOWED : QWS_MASK_NONE;
    r.mask_row = 0;
  }
  DevBufs d;
  qws_batch b;
  memset(&b, 0, sizeof(b));
  b.logits = d.up(logits, (size_t)T * N);
  b.dtype = QWS_DTYPE_F32;
  b.B = T;
  b.V = N;
  b.row_stride = N;
  b.rows = d.up(rows.data(), rows.size());
  b.hist = d.up(hist.data(), hist.size());
  b.drafts = d.up(drafts ? drafts : gen, drafts ? (size_t)(T > 1 ? T - 1 : 0) : 0);
  b.bias_ids = d.up(p->bias_ids, p->n_bias);
  b.bias_vals = d.up(p->bias_vals, p->n_bias);
  b.stop_ids = d.up(p->stop, p->n_stop);
  b.masks = mask.empty() ? nullptr : d.up(mask.data(), mask.size());
  b.mask_words = W;
  b.out_tokens = d.alloc<int>((size_t)T * 4);
  b.out_logits = d.alloc<float>((size_t)T * N * 4);
  const size_t wsb = qws_sample_ws_bytes(T, N);
  void* ws = d.alloc<char>(wsb);
  if (d.err != hipSuccess) return (int)d.err;
  int e = qws_sample(&b, ws, wsb, nullptr);
  if (e == 0) e = (int)hipMemcpy(out, b.out_logits, (size_t)T * N * 4, hipMemcpyDeviceToHost);
  return e;
}

// engine/src/mtp_sample.cu:467-487 (smk_test_dist), dense: out_p[R][N] and the token drawn at (ctr, ST_DRAW).
extern "C" int qws_test_dist(const float* logits, int R, int N, const qws_sampling* cfg, unsigned ctr, float* out_p, int* out_tok) {
  if (!logits || !cfg || R < 1 || N < 8 || (N & 7) || !out_p || !out_tok) return QWS_ERR_INVALID;
  if (!(cfg->temperature > 0.0f) || !(cfg->top_p > 0.0f) || cfg->top_p > 1.0f || !(cfg->min_p >= 0.0f) || cfg->min_p > 1.0f) return QWS_ERR_INVALID;
  qws_row r0;
  const int e0 = qws_row_init(&r0, cfg, nullptr);
  if (e0) return e0;
  r0.position = ctr;
  r0.stream = QWS_ST_DRAW;
  std::vector<qws_row> rows(R, r0);
  DevBufs d;
  qws_batch b;
  memset(&b, 0, sizeof(b));
  b.logits = d.up(logits, (size_t)R * N);
  b.dtype = QWS_DTYPE_F32;
  b.B = R;
  b.V = N;
  b.row_stride = N;
  b.rows = d.up(rows.data(), rows.size());
  b.out_tokens = d.alloc<int>((size_t)R * 4);
  b.out_probs = d.alloc<float>((size_t)R * N * 4);
  const size_t wsb = qws_sample_ws_bytes(R, N);
  void* ws = d.alloc<char>(wsb);
  if (d.err != hipSuccess) return (int)d.err;
  hipError_t he = hipMemset(b.out_probs, 0, (size_t)R * N * 4);
  if (he != hipSuccess) return (int)he;
  int e = qws_sample(&b, ws, wsb, nullptr);
  if (e == 0) e = (int)hipMemcpy(out_p, b.out_probs, (size_t)R * N * 4, hipMemcpyDeviceToHost);
  if (e == 0) e = (int)hipMemcpy(out_tok, b.out_tokens, (size_t)R * 4, hipMemcpyDeviceToHost);
  return e;
}
