#!/usr/bin/env python
"""Benchmark of the MI355X sampling stage (BASELINE.json metric: sampler rows/s at V=248,320, B=1/8/64, and
achieved HBM GB/s against the 8 TB/s peak).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c4,c1,...] [--no-cpu]

A step is one qws_sample call (processors + greedy / min-p / top-k / top-p + Philox draw) over one batch of
synthetic logits already resident in HBM.  The headline workload is config 4 (B=64, fp32, near-flat logits,
top-p 0.95 over the full vocabulary, repetition 1.1 over 4,096-token histories) as a decode step: the histories held
in device state slots built once per request (the reference's proc_begin), each call noting the drawn token and
advancing the row's counters on the device (qws_batch.advance: the reference's proc_note and cycle counter), so that
consecutive calls are consecutive decode steps.  `value` = rows/s of the whole call.  `c4_history` times the same
rows with their histories passed with every call (config.per_call_history in the line).  Each step reads a different copy of the logits (copies together exceed the 256 MB Infinity Cache), so
the timed reads come from HBM, not from cache.  `roofline` is the scan kernel (k_scan, the streaming pass that
reads the logits and histories; the dominant kernel of the call): its algorithmic bytes per launch (logits +
history ids + stop ids + bias pairs + mask words of the batch) / its average launch duration from HIP events
that qws_sample records on its own launch stream during a second timed pass.  `traffic` is the HBM bytes per
k_scan launch measured with rocprofv3 counters (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel of known
size), read from the committed summary profiles/k_scan_c4_traffic.md; null when that file is absent.
`cpu_baseline` times the CPU oracle (oracle/sampler.py) on the same rows on this host: per configuration a warm-up
call and the median of 10 calls, os.cpu_count() threads, the CPU model named.  `rows_with_block_rescans` per
configuration counts the rows whose cut bin was completed by rescanning blocks whose listed window missed that bin
(out_info == 1: one to a few blocks of the row read again by k_resolve; every other row resolves from the first
pass's records alone).
C1 and C2 also carry `host_packed_step_ms` (rows packed on the host every step, then the call) and `graph_step_ms`
(qws_sample + qws_finish_rows replayed from a HIP graph: the step advances on the device).

  python bench.py --copy-calib     # only a 1 GiB device copy, 8 times: the size reference for the counters
  python bench.py --head           # only the quantised head's candidate select + exact rescore (full head shape)
"""
import argparse
import ctypes as C
import json
import math
import os
import sys
import re
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "sampler rows/sec at V=248,320, B=1/8/64; achieved HBM GB/s vs peak"
PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def state_rows(w):
    """The rows of a workload as a decode loop holds them: each row's prompt set and generated counts in a ProcState
    slot built once from its history (qws_state_begin, the reference's proc_begin at admission), the row naming its
    slot instead of carrying the history."""
    import qwen_warp_amd as q
    V = w.logits.shape[1]
    state = q.ProcState(len(w.rows), V)
    rows = []
    for b, r in enumerate(w.rows):
        state.begin(b, r.prompt, r.gen)
        d = {k: getattr(r, k) for k in q.RowSpec.__dataclass_fields__}
        d.update(prompt=[], gen=[], state_slot=b, ngen=len(r.gen) if r.ngen is None else r.ngen)
        rows.append(q.RowSpec(**d))
    return rows, state


def run_config(lib, sampler, w, steps, warmup, decode=False):
    """One configuration's qws_sample calls.  decode=True: the decode loop's step -- rows from state_rows(w), each call
    with qws_batch.advance set (the drawn token noted in the row's slot, ngen and the Philox position advanced on the
    device: the reference's proc_note + cycle counter), so consecutive steps are successive decode steps."""
    import torch
    import qwen_warp_amd as q
    nbytes = w.logits.numel() * w.logits.element_size()
    ncopy = max(2, min(1024, math.ceil(2 * MALL_BYTES / nbytes)))
    lg = w.logits.cuda()
    copies = [lg] + [lg.clone() for _ in range(ncopy - 1)]
    if decode:
        rows, state = state_rows(w)
        packed = q.PackedBatch(rows, w.logits.shape[1], "cuda", state)
    else:
        packed = q.PackedBatch(w.rows, w.logits.shape[1], "cuda")
    out = torch.empty(packed.B, dtype=torch.int32, device="cuda")
    ws = sampler.workspace(packed.B, packed.V)
    batches = [packed.batch(c, out, advance=decode) for c in copies]
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    wsp, wsn = C.c_void_p(ws.data_ptr()), ws.numel()
    fn = lib.qws_sample

    def step(i):
        e = fn(C.byref(batches[i % ncopy]), wsp, wsn, st)
        if e:
            raise RuntimeError(f"qws_sample error {e}")

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # second timed pass: HIP events around each kernel of the call
    lib.qws_timing(1)
    for i in range(steps):
        step(warmup + steps + i)
    a, r, n = C.c_float(), C.c_float(), C.c_int()
    lib.qws_timing_read(C.byref(a), C.byref(r), C.byref(n))
    lib.qws_timing(0)
    torch.cuda.synchronize()
    scan_us, resolve_us = a.value * 1000.0 / n.value, r.value * 1000.0 / n.value
    B = packed.B
    # rows whose cut bin needed rescans of blocks whose listed window missed it (out_info == 1), one call
    info = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    b = packed.batch(copies[0], out, out_info=info, advance=decode)
    e = fn(C.byref(b), wsp, wsn, st)
    if e:
        raise RuntimeError(f"qws_sample error {e}")
    rescan_rows = int((info == 1).sum())
    return dict(B=B, dtype=str(w.logits.dtype).replace("torch.", ""), ms_per_step=ms, rows_per_s=B / (ms / 1000.0), algo_bytes=w.algo_bytes,
                rows_with_block_rescans=rescan_rows,
                step_gbs=w.algo_bytes / (ms / 1000.0) / 1e9, scan_us=scan_us, resolve_us=resolve_us,
                scan_gbs=w.algo_bytes / (scan_us * 1e-6) / 1e9, scan_frac=w.algo_bytes / (scan_us * 1e-6) / 1e9 / PEAK_GBS,
                step_frac=w.algo_bytes / (ms / 1000.0) / 1e9 / PEAK_GBS, copies=ncopy)


def run_decode_step(sampler, w, steps, warmup):
    """A whole decode step of one configuration's rows, two ways (C1 and C2):
    - host: the rows packed on the host each step (PackedBatch from the RowSpecs, the H2D copy of the row array)
      then qws_sample; wall clock over `steps` steps with one synchronisation at the end;
    - graph: the penalties' history held in ProcState slots, one step = qws_sample + qws_finish_rows (notes the
      emitted tokens, advances every row's Philox counter and ngen on the device), captured once in a HIP graph and
      replayed `steps` times (events).
    Both read one logits buffer every step (C1's 1 MB and C2's 4 MB stay in the Infinity Cache), unlike the rotated
    copies of the kernel timing: these are the step costs around the kernels, not an HBM figure."""
    import torch
    import qwen_warp_amd as q
    V = w.logits.shape[1]
    B = w.logits.shape[0]
    lg = w.logits.cuda()
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    sampler.workspace(B, V)
    for i in range(warmup):
        sampler.run(q.PackedBatch(w.rows, V, "cuda"), lg, out_tokens=tok)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        sampler.run(q.PackedBatch(w.rows, V, "cuda"), lg, out_tokens=tok)
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1000.0 / steps
    # device-advancing step in a graph
    state = q.ProcState(B, V)
    rows = []
    for b, r in enumerate(w.rows):
        state.begin(b, r.prompt, r.gen)
        d = {k: getattr(r, k) for k in q.RowSpec.__dataclass_fields__}
        d.update(prompt=[], gen=[], state_slot=b, ngen=len(r.gen) if r.ngen is None else r.ngen)
        rows.append(q.RowSpec(**d))
    packed = q.PackedBatch(rows, V, "cuda", state)
    book = q.StepBook(B)
    for b in range(B):
        book.start(b, 0, -1)
    rs = torch.arange(B, dtype=torch.int32, device="cuda")
    sampler.run(packed, lg, out_tokens=tok)
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        with torch.cuda.graph(graph, stream=cs):
            sampler.run(packed, lg, out_tokens=tok)
            book.finish(rs, tok, state=state, rows=packed)
    torch.cuda.synchronize()
    for i in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return dict(host_packed_step_ms=host_ms, graph_step_ms=e0.elapsed_time(e1) / steps)


def run_verify_config(sampler, w, steps, warmup):
    """Config 3: one qws_verify call (B sequences x K drafts: K + 1 target rows each) per step."""
    import torch
    x = w.extra
    B, K1, V = w.logits.shape
    nbytes = w.logits.numel() * 4
    ncopy = max(2, min(256, math.ceil(2 * MALL_BYTES / nbytes)))
    tl = w.logits.cuda()
    copies = [tl] + [tl.clone() for _ in range(ncopy - 1)]
    dp, dr = x["draft_probs"].cuda(), x["drafts"].cuda()
    inv = sampler.verify_map(x["idmap"].cuda(), V)
    from qwen_warp_amd.sampling import PackedBatch
    packed = PackedBatch(sampler.verify_rows(w.rows, x["drafts"].tolist()), V, "cuda")
    # the first call goes through the checked Python entry point; the timed calls reuse its arguments per copy (the
    # arguments of each call built before timing, as for the sampling configs)
    sampler.verify(copies[0], dp, inv, dr, w.rows, packed)
    calls = [sampler.verify_call(c, dp, inv, dr, packed) for c in copies]
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    fn = sampler.lib.qws_verify

    def step(i):
        vb, ws, _, _ = calls[i % ncopy]
        e = fn(C.byref(vb), ws.data_ptr(), ws.numel(), st)
        if e:
            raise RuntimeError(f"qws_verify error {e}")

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # target rows whose cut bin needed rescans of blocks (out_info == 1 on the target batch), one call
    vb, ws, _, _ = calls[0]
    info = torch.full((B * K1,), -7, dtype=torch.int32, device="cuda")
    vb.target.out_info = info.data_ptr()
    e = fn(C.byref(vb), ws.data_ptr(), ws.numel(), st)
    vb.target.out_info = None
    if e:
        raise RuntimeError(f"qws_verify error {e}")
    rescan_rows = int((info == 1).sum())
    return dict(B=B, K=K1 - 1, rows_with_block_rescans=rescan_rows, dtype="float32", ms_per_step=ms, sequences_per_s=B / (ms / 1000.0), target_rows_per_s=B * K1 / (ms / 1000.0),
                algo_bytes=w.algo_bytes, step_gbs=w.algo_bytes / (ms / 1000.0) / 1e9, copies=ncopy)


def copy_calib(nbytes=1 << 30, reps=8):
    """A plain device copy of known size: the counters' size reference (FETCH_SIZE should read nbytes / 1024 KiB
    per dispatch, WRITE_SIZE the same)."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calib_bytes": nbytes, "reps": reps}), flush=True)


def run_head(steps=50, warmup=5):
    """The quantised head's candidate select + exact rescore (qws_head_select_rescore) at the full head shape
    (N = 248,320 approximate logits per token, K = 5,120, bf16 head rows on the device): one line per (T, R) with the
    average call time over `steps` calls (events; the calls' arguments built before timing).  The timed calls
    rescore into one logits buffer (the select reads it whole; the rescore rewrites R entries per token)."""
    import torch
    from qwen_warp_amd import _lib
    lib = _lib.load()
    N, K = 248320, 5120
    g = torch.Generator(device="cuda").manual_seed(7)
    w = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    ws = torch.empty(lib.qws_head_ws_bytes(), dtype=torch.uint8, device="cuda")
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for T, R in ((1, 20), (1, 64), (16, 20), (16, 64)):
        lg = torch.randn(T, N, device="cuda", generator=g) * 3.0
        x = torch.randn(T, K, device="cuda", generator=g).to(torch.bfloat16)
        tok = torch.empty(T, dtype=torch.int32, device="cuda")
        val = torch.empty(T, dtype=torch.float32, device="cuda")
        args = (C.c_void_p(lg.data_ptr()), C.c_void_p(w.data_ptr()), C.c_void_p(x.data_ptr()), N, K, T, R, C.c_void_p(tok.data_ptr()),
                C.c_void_p(val.data_ptr()), C.c_void_p(ws.data_ptr()), st, None)

        def call():
            e = lib.qws_head_select_rescore(*args)
            if e:
                raise RuntimeError(f"qws_head_select_rescore error {e}")

        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        print(json.dumps({"head_select_rescore": {"T": T, "R": R, "N": N, "K": K, "us_per_call": round(ms * 1000.0, 2)}}), flush=True)


def measured_traffic(path=ROOT / "profiles" / "k_scan_c4_traffic.md"):
    """HBM bytes per k_scan launch on c4 from the committed counter summary (line `traffic_bytes_per_launch: N`)."""
    try:
        m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", path.read_text())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def _cpu_model():
    """The host CPU's model as `lscpu` names it (its "Model name" line), else /proc/cpuinfo's "model name"."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _oracle_procs(S, r):
    if not r.procs_on():
        return None
    return S.RowProcs(presence=r.presence, frequency=r.frequency, repetition=r.repetition, min_tokens=r.min_tokens, prompt=r.prompt, gen=r.gen,
                      ngen=r.ngen, bias=r.bias, allowed=r.allowed, banned=r.banned, stop=r.stop)


def cpu_baseline(wl, reps=10):
    """The CPU oracle (oracle/sampler.py: PyTorch / numpy on the host, exact integer weights) on the same seeded rows:
    for each configuration one warm-up call, then `reps` timed calls (rep i on row i mod B, one sequence of K + 1
    rows for the verify configs); the statistic is the median call time.  Threads: os.cpu_count()."""
    import statistics
    import torch
    from oracle import sampler as S
    ncores = os.cpu_count() or 1
    torch.set_num_threads(ncores)
    per = {}
    for name, w in wl.items():
        if name == "c4_history":  # the same rows as c4 for the oracle
            continue
        if name.startswith("c3"):
            x = w.extra
            B = w.logits.shape[0]

            def call(i, w=w, x=x, B=B):
                b = i % B
                r = w.rows[b]
                S.verify_seq(w.logits[b], x["draft_probs"][b], x["idmap"].numpy(), x["drafts"][b].tolist(), temperature=r.temperature,
                             top_k=r.top_k, top_p=r.top_p, min_p=r.min_p, seed=r.seed, position=r.position, row_key=r.row_key)
            unit, per_call = "sequences/s", 1
        else:
            B = len(w.rows)

            def call(i, w=w, B=B):
                b = i % B
                r = w.rows[b]
                S.sample_row(w.logits[b], r.temperature, r.top_k, r.top_p, r.min_p, r.seed, r.position, r.stream, r.row_key, _oracle_procs(S, r))
            unit, per_call = "rows/s", 1
        call(0)
        ts = []
        for i in range(reps):
            t0 = time.perf_counter()
            call(i + 1)
            ts.append(time.perf_counter() - t0)
        med = statistics.median(ts)
        per[name] = dict(value=per_call / med, unit=unit, median_s=med, reps=reps)
    head = per["c4"]
    return dict(value=head["value"], unit="rows/s", cores=ncores, kind="port", cpu_model=_cpu_model(),
                sample=(f"oracle/sampler.py on c4 rows (V=248,320: processors, top-p 0.95, exact weights, draw), one warm-up then the median "
                        f"of {reps} calls, one row per call, torch threads = os.cpu_count() = {ncores}"),
                per_config=per)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="c4,c1,c1_greedy,c2,c3,c3_aligned,c5")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calib", action="store_true")
    ap.add_argument("--head", action="store_true")
    ap.add_argument("--no-history", action="store_true", help="leave out c4_history (the per-call-history form of c4)")
    ap.add_argument("--batch-sweep", default="", help="comma-separated batch sizes: c4's decode step at each, one JSON line "
                    "per size (the headline line is not printed)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (rows are independent: a larger batch shards by row, one process per GPU); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import qwen_warp_amd as q
    from qwen_warp_amd import _lib, workloads
    torch.cuda.set_device(0)
    if args.copy_calib:
        copy_calib()
        return
    if args.head:
        run_head(args.steps, args.warmup)
        return
    lib = _lib.load()
    sampler = q.Sampler("cuda")
    if args.batch_sweep:  # c4's rows at other batch sizes, as the decode step
        for B in [int(x) for x in args.batch_sweep.split(",") if x]:
            r = run_config(lib, sampler, workloads.c4(B=B), args.steps, args.warmup, decode=True)
            print(json.dumps({"workload": "c4 decode step", **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}}), flush=True)
        return
    names = [c for c in args.configs.split(",") if c]
    if "c4" not in names:
        names = ["c4"] + names
    if "c4_history" not in names and not args.no_history:
        names.insert(names.index("c4") + 1, "c4_history")
    res, wl = {}, {}
    for name in names:
        w = workloads.ALL["c4" if name == "c4_history" else name]()
        wl[name] = w
        if name.startswith("c3"):
            res[name] = run_verify_config(sampler, w, args.steps, args.warmup)
        else:  # c4: the decode step (slots + advance); c4_history: the same rows with their histories passed per call
            res[name] = run_config(lib, sampler, w, args.steps, args.warmup, decode=(name == "c4"))
        if name in ("c1", "c2"):
            res[name].update(run_decode_step(sampler, w, args.steps, args.warmup))
        print(f"# {name}: {json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in res[name].items()})}", file=sys.stderr, flush=True)
    m = res["c4"]
    cpu = None if args.no_cpu else cpu_baseline(wl)
    line = {
        "metric": METRIC, "value": m["rows_per_s"], "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": m["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded; BASELINE.json configs, no checkpoint)",
        "config": {"workload": ("c4: B=64 x V=248,320 fp32 logits ~N(0,0.5), T 1.0, top-k 0, top-p 0.95, repetition 1.1 over 4,096-token "
                                "histories, as a decode step: each row's history in a device state slot built once per request (the "
                                "reference's proc_begin), each call noting the drawn token and advancing the row on the device (proc_note)"),
                   "B": 64, "V": 248320, "algo_bytes_per_call": m["algo_bytes"], "logit_copies_rotated": m["copies"],
                   "per_call_history": None if "c4_history" not in res else {
                       "rows_per_s": res["c4_history"]["rows_per_s"], "ms_per_step": res["c4_history"]["ms_per_step"],
                       "scan_us": res["c4_history"]["scan_us"], "resolve_us": res["c4_history"]["resolve_us"],
                       "note": "the same rows with their 4,096-token histories passed with every call"}},
        "roofline": {"bound": "hbm", "achieved": m["scan_gbs"], "peak": PEAK_GBS, "unit": "GB/s", "frac": m["scan_frac"], "traffic": measured_traffic(),
                     "kernel": "k_scan", "kernel_us": m["scan_us"], "algo_bytes_per_launch": m["algo_bytes"], "resolve_us": m["resolve_us"],
                     "step_gbs": m["step_gbs"], "step_frac": m["step_frac"]},
        "cpu_baseline": cpu,
        "configs": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()} for k, v in res.items()},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
