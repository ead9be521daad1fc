"""The C ABI without a GPU: libqws.so loads, exports every function include/qws.h declares (and the ctypes binding
declares), its struct layouts match the binding's, and its host-only entry points answer (sizes, row defaults,
argument checks that return before any device work)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from qwen_warp_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "qws.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(qws_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_declares_what_the_binding_exports():
    names = header_functions()
    assert len(names) >= 17
    assert names == set(_lib.EXPORTS)


def test_library_exports_every_declared_function(lib):
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_struct_layouts(lib):
    sizes = (C.c_size_t * 4)()
    lib.qws_abi_sizes(sizes)
    assert tuple(sizes) == (C.sizeof(_lib.Sampling), C.sizeof(_lib.Procs), C.sizeof(_lib.Row), C.sizeof(_lib.Batch))
    assert C.sizeof(_lib.Row) == 128


def test_row_init_defaults(lib):
    s = _lib.Sampling(0.7, 20, 0.9, 1, 0.0, 0, 0.0, 0, 5, 0.05)
    r = _lib.Row()
    r.state_slot = 7
    lib.qws_row_init(C.byref(r), C.byref(s), None)
    assert r.state_slot == -1 and r.stream == _lib.ST_FIRST and r.repetition == 1.0 and r.proc_on == 0
    assert abs(r.log2_min_p - (-4.321928094887362)) < 1e-6 and r.top_k == 20 and r.seed == 5


def test_host_size_queries(lib):
    V = 248320
    G = (V + 8191) // 8192
    assert lib.qws_state_bytes(4, V) == 4 * (256 + G * 8192 * 4)
    assert lib.qws_state_bytes(0, V) == 0 and lib.qws_state_bytes(1, 65 * 8192) == 0
    assert lib.qws_sample_ws_bytes(64, V) > 0 and lib.qws_sample_ws_bytes(0, V) == 0


def test_argument_checks_before_device_work(lib):
    assert lib.qws_sample(None, None, 0, None) == _lib.ERR_INVALID
    assert lib.qws_state_begin(None, 1, 248320, 0, None, 0, None, 0, None) == _lib.ERR_INVALID
    assert lib.qws_state_begin(C.c_void_p(256), 1, 248320, 1, None, 0, None, 0, None) == _lib.ERR_INVALID  # slot out of range
    assert lib.qws_state_begin(C.c_void_p(256), 1, 248320, 0, None, 0, None, 70000, None) == _lib.ERR_INVALID  # counts too long
    assert lib.qws_state_note(C.c_void_p(256), 1, 248320, C.c_void_p(256), 1, C.c_void_p(256), 65, None) == _lib.ERR_INVALID  # T > 64
    assert lib.qws_state_note(C.c_void_p(256), 1, 248320, C.c_void_p(256), 0, C.c_void_p(256), 1, None) == _lib.OK  # nothing to do
    b = _lib.Batch()
    b.B, b.V, b.advance = 1, 248320, 1  # a draft pick takes no step: advance is refused before any device work
    assert lib.qws_draft_pick(C.byref(b), C.c_void_p(256), C.c_void_p(256), None, 0, None) == _lib.ERR_INVALID


def test_row_init_pick_matches_draft_row():
    """The C helper qws_row_init_pick (QWS_PICK_DRAFT / FIRST / VERIFY) fills the rows draft_row and the verify rows use."""
    import numpy as np
    import qwen_warp_amd as q
    from oracle import sampler as S
    lib = _lib.load()
    s = q.make_sampling(temperature=0.8, top_k=30, top_p=0.9, draft_sample=1, draft_temperature=1.1, draft_top_k=7, draft_top_p=0.0, seed=5,
                        test_flags=3, min_p=0.05)
    r = _lib.Row()
    lib.qws_row_init_pick(C.byref(r), C.byref(s), None, _lib.PICK_DRAFT, 2)
    d = q.draft_row(temperature=0.8, top_k=30, top_p=0.9, draft_sample=1, draft_temperature=1.1, draft_top_k=7, seed=5, j=2)
    assert (r.temperature, r.top_k, r.top_p, r.min_p, r.proc_on, r.stream, r.draw_word) == \
        (np.float32(d.temperature), d.top_k, np.float32(d.top_p), 0.0, 0, d.stream, 0)
    lib.qws_row_init_pick(C.byref(r), C.byref(s), None, _lib.PICK_FIRST, 0)
    assert r.temperature == 0.0 and r.stream == S.ST_FIRST and r.test_flags == 1  # bit1: keep the argmax; bit0 carries over
    lib.qws_row_init_pick(C.byref(r), C.byref(s), None, _lib.PICK_VERIFY, 3)
    assert r.stream == S.ST_ACCEPT + 3 and r.draw_word == 1 and abs(r.temperature - 0.8) < 1e-7 and abs(r.min_p - 0.05) < 1e-7


def _procs(**kw):
    """A reference smk_procs with repetition on (so that proc_begin's checks apply), plus overrides; arrays kept alive."""
    keep = {}

    def arr(name, typ, vals):
        a = (typ * max(len(vals), 1))(*vals)
        keep[name] = a
        return C.cast(a, C.POINTER(typ)), len(vals)

    base = dict(presence=0.0, frequency=0.0, repetition=1.1, min_tokens=0, prompt=[1, 2], bias_ids=[3], bias_vals=[0.5], allowed=[], stop=[9])
    base.update(kw)
    pr, npr = arr("prompt", C.c_int, base["prompt"])
    bi, nb = arr("bias_ids", C.c_int, base["bias_ids"])
    bv, _ = arr("bias_vals", C.c_float, base["bias_vals"])
    al, na = arr("allowed", C.c_int, base["allowed"])
    st, ns = arr("stop", C.c_int, base["stop"])
    p = _lib.Procs(base["presence"], base["frequency"], base["repetition"], base["min_tokens"], pr, npr, bi, bv, nb, al, na, st, ns)
    p._keep = keep
    return p


@pytest.mark.parametrize("field,value", [
    ("temperature", -0.5), ("temperature", float("nan")), ("temperature", float("inf")),
    ("top_p", 0.0), ("top_p", 1.01), ("top_p", float("nan")),
    ("min_p", -0.01), ("min_p", 1.5),
    ("draft_top_k", -1), ("draft_temperature", -1.0), ("draft_top_p", 1.5), ("draft_top_p", -0.1),
])
def test_row_check_rejects_sampling_fields(lib, field, value):
    """engine/src/mtp_sample.cu:389-392 valid(): each out-of-range field of smk_sampling is QWS_ERR_INVALID, from
    qws_row_check, qws_row_init and qws_row_init_pick alike; the row is then left greedy without processors."""
    s = _lib.Sampling(0.7, 20, 0.9, 1, 0.0, 0, 0.0, 0, 5, 0.0)
    assert lib.qws_row_check(C.byref(s), None, 1000) == _lib.OK
    setattr(s, field, value)
    assert lib.qws_row_check(C.byref(s), None, 1000) == _lib.ERR_INVALID
    r = _lib.Row()
    r.temperature = 3.0
    assert lib.qws_row_init(C.byref(r), C.byref(s), None) == _lib.ERR_INVALID
    assert r.temperature == 0.0 and r.proc_on == 0 and r.state_slot == -1
    assert lib.qws_row_init_pick(C.byref(r), C.byref(s), None, _lib.PICK_VERIFY, 1) == _lib.ERR_INVALID


@pytest.mark.parametrize("kw,err", [
    (dict(repetition=0.0), _lib.ERR_INVALID), (dict(repetition=-1.0), _lib.ERR_INVALID), (dict(repetition=float("nan")), _lib.ERR_INVALID),
    (dict(min_tokens=-1), _lib.ERR_INVALID),
    (dict(prompt=[1, 1000]), _lib.ERR_INVALID), (dict(prompt=[-1]), _lib.ERR_INVALID),
    (dict(bias_ids=[1000], bias_vals=[1.0]), _lib.ERR_INVALID), (dict(allowed=[5, 1000]), _lib.ERR_INVALID), (dict(stop=[1000]), _lib.ERR_INVALID),
    (dict(presence=float("nan")), _lib.ERR_INVALID), (dict(frequency=float("inf")), _lib.ERR_INVALID),
    (dict(bias_ids=[4], bias_vals=[float("nan")]), _lib.ERR_INVALID),
    (dict(bias_ids=list(range(2048)) * 0 + [i % 1000 for i in range(2048)], bias_vals=[0.0] * 2048), _lib.ERR_NOT_SUPPORTED),
])
def test_row_check_rejects_procs_fields(lib, kw, err):
    """engine/src/proc.cu:78-82 proc_begin: ids outside [0, V), repetition <= 0, min_tokens < 0 and too many bias
    entries are rejected; non-finite penalties and bias values as well (a library rule: they would reach the weights)."""
    V = 1000
    assert lib.qws_row_check(None, C.byref(_procs()), V) == _lib.OK
    p = _procs(**kw)
    assert lib.qws_row_check(None, C.byref(p), V) == err
    if "prompt" not in kw and "bias_ids" not in kw and "allowed" not in kw and "stop" not in kw:
        r = _lib.Row()
        assert lib.qws_row_init(C.byref(r), None, C.byref(p)) == err  # no vocabulary there: ranges unchecked
        assert r.proc_on == 0


def test_row_check_null_arrays_and_inactive_processors(lib):
    """A nonzero count needs its array (and bias values); with no processor active nothing is checked, as proc_begin."""
    p = _procs()
    p.prompt = C.POINTER(C.c_int)()
    assert lib.qws_row_check(None, C.byref(p), 1000) == _lib.ERR_INVALID
    p = _procs()
    p.bias_vals = C.POINTER(C.c_float)()
    assert lib.qws_row_check(None, C.byref(p), 1000) == _lib.ERR_INVALID
    p = _procs(repetition=1.0, bias_ids=[], bias_vals=[], prompt=[99999])  # nothing active: the prompt is never read
    assert lib.qws_row_check(None, C.byref(p), 1000) == _lib.OK
    assert lib.qws_row_check(None, None, 0) == _lib.OK
    r = _lib.Row()
    assert lib.qws_row_init(C.byref(r), None, None) == _lib.OK and r.temperature == 0.0 and r.top_p == 1.0


def test_row_init_pick_rejects_kind_and_index(lib):
    s = _lib.Sampling(0.7, 20, 0.9, 1, 0.0, 0, 0.0, 0, 5, 0.0)
    r = _lib.Row()
    assert lib.qws_row_init_pick(C.byref(r), C.byref(s), None, 7, 0) == _lib.ERR_INVALID
    assert lib.qws_row_init_pick(C.byref(r), C.byref(s), None, _lib.PICK_DRAFT, 0) == _lib.ERR_INVALID  # drafts count from 1
    assert lib.qws_row_init_pick(C.byref(r), C.byref(s), None, _lib.PICK_DRAFT, 1) == _lib.OK and r.stream == _lib.ST_DRAFT + 1


def test_new_entry_argument_checks(lib):
    """qws_state_read, qws_finish_forced and qws_timing_read_verify reject bad arguments before any device work."""
    assert lib.qws_state_read(None, 1, 248320, 0, C.c_void_p(256), None, None) == _lib.ERR_INVALID
    assert lib.qws_state_read(C.c_void_p(256), 1, 248320, 1, C.c_void_p(256), None, None) == _lib.ERR_INVALID  # slot out of range
    assert lib.qws_state_read(C.c_void_p(256), 1, 248320, 0, None, None, None) == _lib.ERR_INVALID  # no counts array
    args = [C.c_void_p(256), 1, C.c_void_p(256), 8, C.c_void_p(256), 1, C.c_void_p(256), None, 1, None, 0, 0, None, 0, 0, None, 1]
    assert lib.qws_finish_forced(*args, None, 2, None) == _lib.ERR_INVALID  # a schedule length without a schedule
    assert lib.qws_finish_forced(*args, C.c_void_p(256), -1, None) == _lib.ERR_INVALID
    assert lib.qws_timing_read_verify(None, None, None) == _lib.ERR_INVALID
