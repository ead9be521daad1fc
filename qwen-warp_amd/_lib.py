"""ctypes binding of libqws.so (include/qws.h).

The library must be built (qwen-warp_amd/build.py, or __graft_entry__.build()); loading fails loudly
otherwise -- there is no CPU fallback.  The error convention is the reference's (engine/smk.py:48-50):
a nonzero status raises RuntimeError.
"""
import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libqws.so"

OK, ERR_INVALID, ERR_NOT_SUPPORTED = 0, 1, 801
NOALLOC_SCRATCH_BYTES = 16 << 20  # include/qws.h QWS_NOALLOC_SCRATCH_BYTES
DTYPE_F32, DTYPE_BF16 = 0, 1
MASK_NONE, MASK_BANNED, MASK_ALLOWED = 0, 1, 2
ST_ACCEPT, ST_DRAFT, ST_FIRST, ST_DRAW = 0x1000, 0x2000, 0x3000, 0x4000
TF_BROKEN, TF_RESCAN, TF_STAGED_DRAW, TF_SPLIT_SELECT = 1, 2, 4, 8  # qws_row.test_flags (include/qws.h QWS_TF_*)
PICK_FIRST, PICK_DRAFT, PICK_VERIFY, PICK_DRAW = 0, 1, 2, 3  # qws_row_init_pick kinds (include/qws.h QWS_PICK_*)


class Sampling(C.Structure):
    """include/qws.h qws_sampling == the reference's smk_sampling (engine/include/mtp.h:97-108, engine/spec.py:40-42)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("draft_sample", C.c_int),
                ("draft_temperature", C.c_float), ("draft_top_k", C.c_int), ("draft_top_p", C.c_float),
                ("test_flags", C.c_int), ("seed", C.c_ulonglong), ("min_p", C.c_float)]


class Procs(C.Structure):
    """include/qws.h qws_procs == the reference's smk_procs (engine/include/engine.h:142-154, engine/spec.py:49-53)."""
    _fields_ = [("presence", C.c_float), ("frequency", C.c_float), ("repetition", C.c_float), ("min_tokens", C.c_int),
                ("prompt", C.POINTER(C.c_int)), ("n_prompt", C.c_int), ("bias_ids", C.POINTER(C.c_int)),
                ("bias_vals", C.POINTER(C.c_float)), ("n_bias", C.c_int), ("allowed", C.POINTER(C.c_int)),
                ("n_allowed", C.c_int), ("stop", C.POINTER(C.c_int)), ("n_stop", C.c_int)]


class Row(C.Structure):
    """include/qws.h qws_row: one logits row of a batched call (device memory)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("log2_min_p", C.c_double), ("seed", C.c_ulonglong), ("position", C.c_uint), ("stream", C.c_uint),
                ("row_key", C.c_uint), ("proc_on", C.c_int), ("presence", C.c_float), ("frequency", C.c_float),
                ("repetition", C.c_float), ("min_tokens", C.c_int), ("ngen", C.c_int), ("hist_off", C.c_int),
                ("n_prompt", C.c_int), ("n_gen", C.c_int), ("draft_off", C.c_int), ("n_drafts", C.c_int),
                ("bias_off", C.c_int), ("n_bias", C.c_int), ("stop_off", C.c_int), ("n_stop", C.c_int),
                ("mask_mode", C.c_int), ("mask_row", C.c_int), ("test_flags", C.c_int), ("draw_word", C.c_int),
                ("state_slot", C.c_int), ("pad_", C.c_int)]


class Batch(C.Structure):
    """include/qws.h qws_batch."""
    _fields_ = [("logits", C.c_void_p), ("dtype", C.c_int), ("B", C.c_int), ("V", C.c_int), ("row_stride", C.c_longlong),
                ("rows", C.c_void_p), ("hist", C.c_void_p), ("drafts", C.c_void_p), ("bias_ids", C.c_void_p),
                ("bias_vals", C.c_void_p), ("stop_ids", C.c_void_p), ("masks", C.c_void_p), ("mask_words", C.c_int),
                ("out_tokens", C.c_void_p), ("out_logits", C.c_void_p), ("out_probs", C.c_void_p), ("out_info", C.c_void_p),
                ("state_mem", C.c_void_p), ("state_slots", C.c_int), ("advance", C.c_int)]


class VerifyBatch(C.Structure):
    """include/qws.h qws_verify_batch."""
    _fields_ = [("target", Batch), ("B", C.c_int), ("K", C.c_int), ("Vd", C.c_int), ("draft_tokens", C.c_void_p), ("draft_probs", C.c_void_p),
                ("inv_map", C.c_void_p), ("out_tokens", C.c_void_p), ("out_n", C.c_void_p), ("n_chain", C.c_void_p)]


class Seq(C.Structure):
    """include/qws.h qws_seq: a sequence's decode-step bookkeeping (device memory)."""
    _fields_ = [("pos", C.c_int), ("last", C.c_int), ("outn", C.c_int), ("cycles", C.c_int), ("hist", C.c_int * 8)]


class PldCfg(C.Structure):
    """include/qws.h qws_pld_cfg == the reference's smk_pld_cfg (engine/include/pld.h:13-20)."""
    _fields_ = [(k, C.c_int) for k in ("n", "min_len", "max_tail", "cap", "back", "longest")]


EXPORTS = ("qws_sample_ws_bytes", "qws_sample", "qws_sample_noalloc", "qws_verify_ws_bytes", "qws_verify", "qws_verify_map", "qws_draft_pick",
           "qws_row_init_pick", "qws_argmax_ws_bytes", "qws_argmax",
           "qws_state_bytes", "qws_state_begin", "qws_state_note", "qws_state_read",
           "qws_finish", "qws_finish_rows", "qws_finish_forced", "qws_head_ws_bytes", "qws_head_select_rescore", "qws_head_ws_cand", "qws_head_ws_exact", "qws_pld_default_cfg", "qws_pld_bytes", "qws_pld_reset", "qws_pld_append", "qws_pld_propose",
           "qws_row_init", "qws_row_check", "qws_abi_sizes",
           "qws_timing", "qws_timing_read", "qws_timing_read_verify", "qws_test_philox", "qws_test_proc_logits", "qws_test_dist")

_LIB = None


def load(path=None):
    """Loads libqws.so once, declares the signatures and checks the struct layouts."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"libqws.so not built ({p}); run python qwen-warp_amd/build.py")
    lib = C.CDLL(str(p))
    vp, ci, cu, sz = C.c_void_p, C.c_int, C.c_uint, C.c_size_t
    lib.qws_sample_ws_bytes.argtypes, lib.qws_sample_ws_bytes.restype = [ci, ci], sz
    lib.qws_sample.argtypes, lib.qws_sample.restype = [C.POINTER(Batch), vp, sz, vp], ci
    lib.qws_sample_noalloc.argtypes, lib.qws_sample_noalloc.restype = [C.POINTER(Batch), vp], ci
    lib.qws_verify_ws_bytes.argtypes, lib.qws_verify_ws_bytes.restype = [ci, ci, ci], sz
    lib.qws_verify.argtypes, lib.qws_verify.restype = [C.POINTER(VerifyBatch), vp, sz, vp], ci
    lib.qws_verify_map.argtypes, lib.qws_verify_map.restype = [vp, ci, ci, vp, vp], ci
    lib.qws_draft_pick.argtypes, lib.qws_draft_pick.restype = [C.POINTER(Batch), vp, vp, vp, sz, vp], ci
    lib.qws_row_init_pick.argtypes = [C.POINTER(Row), C.POINTER(Sampling), C.POINTER(Procs), ci, ci]
    lib.qws_row_init_pick.restype = ci
    lib.qws_row_check.argtypes, lib.qws_row_check.restype = [C.POINTER(Sampling), C.POINTER(Procs), ci], ci
    lib.qws_state_bytes.argtypes, lib.qws_state_bytes.restype = [ci, ci], sz
    lib.qws_state_begin.argtypes, lib.qws_state_begin.restype = [vp, ci, ci, ci, vp, ci, vp, ci, vp], ci
    lib.qws_state_note.argtypes, lib.qws_state_note.restype = [vp, ci, ci, vp, ci, vp, ci, vp], ci
    lib.qws_state_read.argtypes, lib.qws_state_read.restype = [vp, ci, ci, ci, vp, vp, vp], ci
    lib.qws_finish.argtypes = [vp, ci, vp, ci, vp, ci, vp, vp, ci, vp, ci, ci, vp, ci, ci, vp]
    lib.qws_finish.restype = ci
    lib.qws_finish_rows.argtypes = [vp, ci, vp, ci, vp, ci, vp, vp, ci, vp, ci, ci, vp, ci, ci, vp, ci, vp]
    lib.qws_finish_rows.restype = ci
    lib.qws_finish_forced.argtypes = [vp, ci, vp, ci, vp, ci, vp, vp, ci, vp, ci, ci, vp, ci, ci, vp, ci, vp, ci, vp]
    lib.qws_finish_forced.restype = ci
    lib.qws_head_ws_bytes.argtypes, lib.qws_head_ws_bytes.restype = [], sz
    lib.qws_head_select_rescore.argtypes = [vp, vp, vp, ci, ci, ci, ci, vp, vp, vp, vp, vp]
    lib.qws_head_select_rescore.restype = ci
    lib.qws_head_ws_cand.argtypes, lib.qws_head_ws_cand.restype = [vp], vp
    lib.qws_head_ws_exact.argtypes, lib.qws_head_ws_exact.restype = [vp], vp
    lib.qws_pld_default_cfg.argtypes, lib.qws_pld_default_cfg.restype = [C.POINTER(PldCfg)], None
    lib.qws_pld_bytes.argtypes, lib.qws_pld_bytes.restype = [ci, ci], sz
    lib.qws_pld_reset.argtypes, lib.qws_pld_reset.restype = [vp, ci, ci, ci, vp, ci, vp], ci
    lib.qws_pld_append.argtypes, lib.qws_pld_append.restype = [vp, ci, ci, vp, ci, vp, ci, vp], ci
    lib.qws_pld_propose.argtypes = [vp, ci, ci, C.POINTER(PldCfg), vp, ci, vp, ci, ci, ci, vp, vp, vp, vp]
    lib.qws_pld_propose.restype = ci
    lib.qws_argmax_ws_bytes.argtypes, lib.qws_argmax_ws_bytes.restype = [], sz
    lib.qws_argmax.argtypes, lib.qws_argmax.restype = [vp, ci, ci, vp, vp, vp, vp], ci
    lib.qws_row_init.argtypes, lib.qws_row_init.restype = [C.POINTER(Row), C.POINTER(Sampling), C.POINTER(Procs)], ci
    lib.qws_abi_sizes.argtypes, lib.qws_abi_sizes.restype = [C.POINTER(C.c_size_t)], None
    lib.qws_timing.argtypes, lib.qws_timing.restype = [ci], ci
    lib.qws_timing_read.argtypes = [C.POINTER(C.c_float), C.POINTER(C.c_float), C.POINTER(ci)]
    lib.qws_timing_read.restype = ci
    lib.qws_timing_read_verify.argtypes = [C.POINTER(C.c_float), C.POINTER(C.c_float), C.POINTER(ci)]
    lib.qws_timing_read_verify.restype = ci
    lib.qws_test_philox.argtypes, lib.qws_test_philox.restype = [C.POINTER(cu), C.POINTER(cu), C.POINTER(cu)], ci
    lib.qws_test_proc_logits.argtypes = [C.POINTER(Procs), ci, ci, C.POINTER(ci), ci, C.POINTER(ci), vp, vp]
    lib.qws_test_proc_logits.restype = ci
    lib.qws_test_dist.argtypes, lib.qws_test_dist.restype = [vp, ci, ci, C.POINTER(Sampling), cu, vp, vp], ci
    sizes = (C.c_size_t * 4)()
    lib.qws_abi_sizes(sizes)
    want = (C.sizeof(Sampling), C.sizeof(Procs), C.sizeof(Row), C.sizeof(Batch))
    if tuple(sizes) != want:
        raise RuntimeError(f"libqws ABI mismatch: library {tuple(sizes)} vs binding {want}")
    if path is None:
        _LIB = lib
    return lib


def check(err, what=""):
    """engine/smk.py:48-50: a nonzero status is an error."""
    if err != 0:
        raise RuntimeError(f"{what}: qws/hip error {err}")
