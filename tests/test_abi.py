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
