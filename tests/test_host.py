"""Host-side request handling without a GPU: the request validation the reference's server answers with HTTP 400
(its cases restated from tests/test_sampling_params.py:209-226 and the top_k rules of tests/test_server_seed.py:10-11,
with the limits of docs/USAGE.md:80-87), GenParams.procs() gating (server/smk_runner.py:71-76), the request -> row
mapping (server/smk_runner.py:597-607) and the make_sampling / make_procs defaults (engine/spec.py:45-67)."""
import ctypes as C

import pytest

import qwen_warp_amd as q

EOS = (248044, 248046)  # the reference tests' EOS pair (tests/test_logit_procs.py:112)


def params(**kw):
    base = dict(max_tokens=8, temperature=0.7, min_tokens_ids=frozenset(EOS))
    base.update(kw)
    return q.GenParams(**base)


def rejects(param, **kw):
    with pytest.raises(q.ValidationError) as e:
        q.check_supported(params(**kw))
    assert e.value.parameter == param, (param, e.value.parameter, str(e.value))


@pytest.mark.parametrize("name,param,kw", [
    ("presence_penalty 3", "presence_penalty", dict(presence_penalty=3.0)),
    ("frequency_penalty -2.5", "frequency_penalty", dict(frequency_penalty=-2.5)),
    ("repetition_penalty 0", "repetition_penalty", dict(repetition_penalty=0.0)),
    ("min_p 1.5", "min_p", dict(min_p=1.5)),
    ("min_tokens above max_tokens", "min_tokens", dict(min_tokens=20)),
    ("logit_bias with an out-of-vocabulary id", "logit_bias", dict(logit_bias={"300000": 1.0})),
    ("logit_bias with a non-integer key", "logit_bias", dict(logit_bias={"abc": 1.0})),
    ("logit_bias with 1025 entries", "logit_bias", dict(logit_bias={str(i): 1.0 for i in range(1025)})),
    ("empty allowed_token_ids", "allowed_token_ids", dict(allowed_token_ids=())),
    ("allowed_token_ids with an out-of-vocabulary id", "allowed_token_ids", dict(allowed_token_ids=(5, 999999))),
    ("allowed_token_ids made of stop tokens only + min_tokens", "min_tokens", dict(allowed_token_ids=EOS, min_tokens=3)),
])
def test_reference_400_cases(name, param, kw):
    """tests/test_sampling_params.py:214-224: each request is rejected, naming the parameter."""
    rejects(param, **kw)


def test_reference_accepted_limits():
    q.check_supported(params(logit_bias={str(i): 1.0 for i in range(1024)}))  # exactly 1,024 entries (test_sampling_params.py:225)
    q.check_supported(params(presence_penalty=2.0, frequency_penalty=-2.0, min_tokens=8, min_p=1.0, top_p=1.0))
    q.check_supported(params(allowed_token_ids=EOS + (7,), min_tokens=3))  # a non-stop token is allowed
    q.check_supported(params(allowed_token_ids=EOS))  # stop tokens only, without min_tokens


@pytest.mark.parametrize("k", [-1, 0, 1, 20, 64])
def test_top_k_accepted(k):
    """tests/test_server_seed.py:10-11: -1, 0, 1, 20 and 64 are accepted with the reference's 64-candidate cap."""
    q.check_supported(params(top_k=k, cap64=True))
    q.check_supported(params(top_k=k))


@pytest.mark.parametrize("k", [65, 1000])
def test_top_k_above_the_cap(k):
    """tests/test_server_seed.py:11: 65 and 1000 give HTTP 400 naming top_k and the limit; without the cap (the
    full-vocabulary semantics) they are ordinary top-k values."""
    with pytest.raises(q.ValidationError) as e:
        q.check_supported(params(top_k=k, cap64=True))
    assert e.value.parameter == "top_k" and "64" in str(e.value)
    q.check_supported(params(top_k=k))


def test_other_parameter_limits():
    rejects("top_k", top_k=-2)
    rejects("temperature", temperature=-0.1)
    rejects("temperature", temperature=float("inf"))
    rejects("top_p", top_p=0.0)
    rejects("top_p", top_p=1.5)
    rejects("min_p", min_p=-0.1)
    rejects("repetition_penalty", repetition_penalty=float("nan"))
    rejects("min_tokens", min_tokens=-1)
    rejects("logit_bias", logit_bias={5: float("inf")})
    rejects("logit_bias", logit_bias={-1: 1.0})


def test_procs_gating():
    """server/smk_runner.py:71-76: no processor arguments when none is active; min_p is a sampler parameter."""
    assert q.GenParams(temperature=0.7, min_p=0.1).procs([1, 2]) is None
    assert q.GenParams(repetition_penalty=1.0, presence_penalty=0.0).procs([1]) is None
    for kw in (dict(presence_penalty=0.5), dict(frequency_penalty=-0.5), dict(repetition_penalty=1.1), dict(min_tokens=2),
               dict(logit_bias={3: 1.0}), dict(allowed_token_ids=(1, 2))):
        pr = q.GenParams(min_tokens_ids=frozenset({9, 4}), **kw).procs([5, 6])
        assert pr is not None and pr["prompt"] == [5, 6] and pr["stop"] == [4, 9]


def test_request_to_row():
    """server/smk_runner.py:597-607 with the two top-k semantics, the seed default and the bias clamp."""
    r = q.row_from_params(q.GenParams(temperature=0.8, top_k=0, top_p=0.9, seed=7), gen_ids=[3], position=5, row_key=2)
    assert (r.temperature, r.top_k, r.top_p, r.seed, r.position, r.row_key, r.gen) == (0.8, 0, 0.9, 7, 5, 2, [3])
    assert q.row_from_params(q.GenParams(temperature=0.8, top_k=-1, cap64=True)).top_k == 64  # <= 0: the 64 best candidates
    assert q.row_from_params(q.GenParams(temperature=0.8, top_k=20, cap64=True)).top_k == 20
    seeds = {q.row_from_params(q.GenParams(temperature=1.0)).seed for _ in range(8)}
    assert len(seeds) > 1 and all(0 <= s < 2 ** 62 for s in seeds)  # a fresh 62-bit seed per request
    g = q.row_from_params(q.GenParams(temperature=0.0, top_k=5, repetition_penalty=1.2, logit_bias={"7": 250.0, 8: -1e9, 9: 0.5}), prompt_ids=[1, 2])
    assert g.temperature == 0.0 and g.repetition == 1.2 and g.prompt == [1, 2]
    assert g.bias == {7: 100.0, 8: -100.0, 9: 0.5}  # integer ids, values clamped to [-100, 100]
    with pytest.raises(q.ValidationError):
        q.row_from_params(q.GenParams(temperature=0.5, top_p=0.0))


def test_reference_struct_defaults():
    """engine/spec.py:45-67: make_sampling / make_procs defaults and field order."""
    s = q.make_sampling()
    assert (s.temperature, s.top_k, s.top_p, s.draft_sample, s.draft_temperature, s.draft_top_k, s.draft_top_p, s.test_flags, s.seed) == \
        (0.0, 20, 1.0, 1, 0.0, 0, 0.0, 0, 0)
    assert abs(s.min_p) == 0.0
    p, keep = q.make_procs()
    assert (p.presence, p.frequency, p.repetition, p.min_tokens, p.n_prompt, p.n_bias, p.n_allowed, p.n_stop) == (0.0, 0.0, 1.0, 0, 0, 0, 0, 0)
    p, keep = q.make_procs(prompt=[4, 5], bias={10: 1.5, 11: -2.0}, allowed=[1, 2, 3], stop=EOS, min_tokens=2)
    assert (p.n_prompt, p.n_bias, p.n_allowed, p.n_stop, p.min_tokens) == (2, 2, 3, 2, 2)
    assert [p.bias_ids[i] for i in range(2)] == [10, 11] and [p.bias_vals[i] for i in range(2)] == [1.5, -2.0]
    assert [p.stop[i] for i in range(2)] == list(EOS) and isinstance(p.prompt, C.POINTER(C.c_int))


def test_packed_batch_id_containers():
    """Histories, stop ids and allowed lists given as lists, tuples, sets, numpy arrays or tensors pack to the same
    device bytes; an empty allowed list masks nothing; an id outside [0, V) is rejected whatever the container."""
    import numpy as np
    import torch
    V = 4096
    ids = [5, 7, 9, 4000]

    def packed(conv):
        rows = [q.RowSpec(prompt=conv([1, 2]), gen=conv(ids), stop=conv([3]), allowed=conv(ids), drafts=conv([8, 9]), min_tokens=1),
                q.RowSpec(gen=conv([]), allowed=conv([]), repetition=1.1)]
        return q.PackedBatch(rows, V, "cpu")

    want = packed(list)
    for conv in (tuple, np.array, torch.tensor, lambda a: np.array(a, dtype=np.int32)):
        got = packed(conv)
        assert torch.equal(got.dev_buf, want.dev_buf)
    assert want.host_rows[1].mask_mode == 0 and want.masks_t.shape == (1, (V + 31) // 32)
    s = q.PackedBatch([q.RowSpec(allowed=set(ids))], V, "cpu")
    assert sorted(np.nonzero(np.unpackbits(s.masks_t.numpy().view(np.uint8), bitorder="little"))[0].tolist()) == ids
    for conv in (list, np.array, torch.tensor):
        with pytest.raises(q.ValidationError):
            q.PackedBatch([q.RowSpec(gen=conv([1, V]))], V, "cpu")
        with pytest.raises(q.ValidationError):
            q.PackedBatch([q.RowSpec(allowed=conv([-1]))], V, "cpu")
    # ids that are not integers are refused whatever the container (never truncated: 3.7 is not token 3)
    for bad in ([3.7, 1], np.array([3.7, 1.0]), torch.tensor([3.7, 1.0]), np.array([True, False]), torch.tensor([True]), [True], ["5"],
                [1, True], (np.int32(3), 2.0), {4, 5.5}):
        with pytest.raises(q.ValidationError):
            q.PackedBatch([q.RowSpec(gen=bad, repetition=1.1)], V, "cpu")
    assert torch.equal(packed(lambda a: np.array(a, dtype=np.int64)).dev_buf, want.dev_buf)


def test_advance_refuses_penalties_without_state():
    """A step taken on the device (qws_batch.advance, qws_finish_rows) cannot extend a CSR history: rows whose penalties
    count generated tokens must keep them in a state slot; other rows (bias, min_tokens, masks, no processors) may."""
    import torch
    V = 4096
    for kw in (dict(repetition=1.1), dict(presence=0.5), dict(frequency=0.3), dict(repetition=1.1, gen=[1, 2]), dict(repetition=1.2, prompt=[5])):
        pb = q.PackedBatch([q.RowSpec(temperature=1.0, **kw)], V, "cpu")
        with pytest.raises(q.ValidationError):
            pb.batch(torch.zeros(1, V), torch.zeros(1, dtype=torch.int32), advance=True)
        with pytest.raises(q.ValidationError):
            pb.check_advance()
    for kw in (dict(), dict(bias={3: 1.0}), dict(min_tokens=2, stop=[7]), dict(allowed=[1, 2, 3])):
        pb = q.PackedBatch([q.RowSpec(temperature=1.0, **kw)], V, "cpu")
        pb.check_advance()
    # with a state slot the same penalties may advance
    class _State:
        V, slots = 4096, 2
        mem = torch.zeros(1)
    pb = q.PackedBatch([q.RowSpec(temperature=1.0, repetition=1.1, state_slot=0)], V, "cpu", state=_State())
    pb.check_advance()
