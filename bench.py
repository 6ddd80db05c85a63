"""Benchmark of the batched sampling step on one MI355X.

Workload (default): config C3 of the contract — B=256 rows, V=151936 fp32 logits
~N(0,3^2) with 0.1% of entries from N(8,2^2), top-k 50, top-p 0.95, T 0.7,
repetition 1.1 / presence 0.5 / frequency 0.3 over 2048-token Zipf(1.1)
histories, one caller uniform per row.  A step = one llmk_sample_batch call
over the whole batch with every input already resident in HBM.  Several
copies of the logits are rotated so that consecutive steps do not re-read the
previous step's logits from the 256 MB Infinity Cache.

Prints ONE JSON line on stdout.  Extra diagnostics go to stderr.
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llm-rs_amd"))
sys.path.insert(0, ROOT)

METRIC = "sampled tokens/sec and µs/step at B=256, V=151936 fp32; % HBM roofline"
HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 << 20


def kernel_source_digest():
    """sha256 of the sampling kernel's source: a traffic summary applies to the
    kernel it was measured on and to no later edit."""
    import hashlib
    with open(os.path.join(ROOT, "llm-rs_amd", "csrc", "llmk_sampler.hip"), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def measured_traffic(config):
    """HBM bytes per call (the sampling launch and the one after it) from the
    committed counter summary (FETCH_SIZE + WRITE_SIZE, scaled by a plain
    copy), or None when there is none or it was measured on another version
    of the kernels."""
    import re
    path = os.path.join(ROOT, "profiles", f"stream_kernel_{config}_hbm_traffic.md")
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None, "no counter summary"
    m = re.search(r"^traffic_bytes_per_launch = (\d+)$", text, re.M)
    d = re.search(r"^kernel_source_sha256 = ([0-9a-f]{64})$", text, re.M)
    if not m:
        return None, "no traffic line in " + os.path.basename(path)
    if not d or d.group(1) != kernel_source_digest():
        return None, "counter summary measured on another version of llmk_sampler.hip"
    return int(m.group(1)), os.path.basename(path)


def with_count_history(w, db):
    """db with each row's history in the count-table form (hist_counts): its
    distinct tokens, ascending, with their occurrences, as the device push
    llmk_history_count_append keeps them."""
    import numpy as np
    import torch
    toks, cnts = [], []
    for b in range(w.B):
        u, c = np.unique(w.hist_tokens[w.hist_offsets[b]:w.hist_offsets[b + 1]],
                         return_counts=True)
        toks.append(u.astype(np.uint32))
        cnts.append(c.astype(np.uint32))
    offs = np.concatenate([[0], np.cumsum([len(u) for u in toks])]).astype(np.uint32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(db.logits.device)
    db.hist_offsets = T(offs)
    db.hist_tokens = T(np.concatenate(toks))
    db.hist_counts = T(np.concatenate(cnts))
    return db, int(offs[-1])


def rotated_sets(llmk, db0, logit_bytes, sets=0):
    """db0 and clones of its logits, enough that consecutive steps do not
    find the previous step's logits in the 256 MB MALL."""
    import numpy as np
    nsets = sets or max(1, int(np.ceil(2 * MALL_BYTES / logit_bytes)) + 1)
    dbs = [db0]
    for _ in range(nsets - 1):
        d = llmk.DeviceBatch(**{k: getattr(db0, k) for k in db0.__dataclass_fields__})
        d.logits = db0.logits.clone()
        dbs.append(d)
    return dbs


def back_to_back(torch, s, prepared, K, stream):
    """K calls of llmk_sample_batch, rotating over the prepared argument
    sets, between two events on the launch stream: the time per call (its
    sampling launch, and the launch after it that finishes rows whose band
    check failed, when the call has top-k and 16 rows or more)."""
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(K):
        s.launch_prepared(prepared[i % len(prepared)], stream)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / K


def time_config(llmk, synth, torch, name, steps=20, warmup=5):
    """Time per launch of one config (back-to-back launches between two
    events), its logits rotated over enough copies to leave the MALL."""
    import numpy as np
    counts = name.endswith("-counts")
    if counts:
        name = name[:-7]
    if name.endswith("-f16"):
        # the config with its logits rounded to f16 (a half-precision lm_head
        # output handed over as it is)
        w = synth.make(name[:-4])
        h = w.logits.astype(np.float16)
        w.bf16_bits, w.logits, w.dtype = h.view(np.uint16), h.astype(np.float32), "f16"
        w.name = name
    elif "-seed" in name:
        # the config drawn from another seed of its generator (the seeded C3
        # batch holds one row whose band check fails: 1 of 256, where 1024
        # rows of other seeds hold none)
        base, seed = name.split("-seed")
        w = synth.make(base, seed=int(seed))
        w.name = name
    else:
        w = synth.make(name)
    db0 = w.to_device()
    alg = w.algorithmic_bytes()
    if counts:
        # the history read as (token, count) pairs: 8 bytes per distinct token
        db0, nd = with_count_history(w, db0)
        alg += 8 * nd - 4 * int(w.hist_tokens.size)
    dbs = rotated_sets(llmk, db0, db0.logits.numel() * db0.logits.element_size())
    s = llmk.HipSampler(max_batch=w.B, max_vocab=w.V)
    tok = torch.empty(w.B, dtype=torch.int32, device="cuda:0")
    prepared = [s.prepare(d, tok) for d in dbs]
    stream = torch.cuda.current_stream()
    back_to_back(torch, s, prepared, warmup, stream)
    us = back_to_back(torch, s, prepared, steps, stream) * 1e3
    gbps = alg / (us * 1e-6) / 1e9
    s.close()
    return {"B": w.B, "V": w.V, "dtype": w.dtype, "us_per_step": us,
            "tokens_per_s": w.B / (us * 1e-6), "achieved_GBps": gbps,
            "frac_of_8TBps": gbps / HBM_PEAK_GBPS}


def time_mask(llmk, synth, torch, op, steps=3):
    """The mask forms in place: apply_top_k at C3's shape (k 50) and apply_top_p
    at C4's (top-p 0.9).  Each launch masks a freshly restored copy of the
    logits, restored before all timed launches of a round so that it has left
    the MALL; the launches of a round run back to back between two events on
    the launch stream."""
    import numpy as np
    w = synth.make("C3" if op == "top_k" else "C4")
    src = torch.from_numpy(w.logits).to("cuda:0")
    nbytes = src.numel() * 4
    nsets = max(1, int(np.ceil(2 * MALL_BYTES / nbytes)) + 1)
    bufs = [torch.empty_like(src) for _ in range(nsets)]
    s = llmk.HipSampler(max_batch=w.B, max_vocab=w.V)
    if op == "top_k":
        par = torch.full((w.B,), 50, dtype=torch.int32, device="cuda:0")
        call = lambda t: s.apply_top_k(t, par)
    else:
        par = torch.from_numpy(w.top_p).to("cuda:0")
        call = lambda t: s.apply_top_p(t, par)
    stream = torch.cuda.current_stream()
    times = []
    for r in range(steps + 1):
        for b in bufs:
            b.copy_(src)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for b in bufs:
            call(b)
        e1.record(stream)
        torch.cuda.synchronize()
        if r:  # the first round warms up
            times.append(e0.elapsed_time(e1) / len(bufs))
    masked = int((bufs[0] != src).sum().item())
    us = float(np.mean(times)) * 1e3
    alg = nbytes + 4 * masked + 4 * w.B
    gbps = alg / (us * 1e-6) / 1e9
    s.close()
    return {"op": op, "B": w.B, "V": w.V, "param": 50 if op == "top_k" else float(w.top_p[0]),
            "us_per_call": us, "masked_per_row": masked / w.B,
            "algorithmic_bytes": alg, "achieved_GBps": gbps, "frac_of_8TBps": gbps / HBM_PEAK_GBPS}


def stream_read_gbps(torch, nbytes=2 << 30, reps=5):
    """The box's achievable streaming-read bandwidth: llmk_read_probe (every
    lane reads 128-bit words with non-temporal loads, as the sampler does)
    over nbytes, best over a few grid sizes and repetitions."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "llm-rs_amd", "llmk", "libllmk_read_probe.so"))
    lib.llmk_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                    ctypes.c_uint32, ctypes.c_void_p]
    x = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    out = torch.zeros(1, dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream()
    best = 0.0
    for blocks in (512, 1024, 2048):
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            rc = lib.llmk_read_probe(x.data_ptr(), nbytes, out.data_ptr(), blocks,
                                     ctypes.c_void_p(stream.cuda_stream))
            b.record(stream)
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError(f"llmk_read_probe failed: {rc}")
            best = max(best, nbytes / (a.elapsed_time(b) * 1e-3) / 1e9)
    del x
    return best


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(w, budget_s=12.0):
    """The oracle's `ref` mode (a C restatement of llm-core/src/sampler.rs
    sample_logits, full-vocabulary sort per row) timed on this host: rows
    serial on one core, as Scheduler::step calls it (scheduler.rs:138-145)."""
    import numpy as np
    from oracle import llmk_oracle as O
    O.load()
    rows_done, t_total = 0, 0.0
    order = np.arange(w.B)
    while t_total < budget_s and rows_done < 4 * w.B:
        sel = order[rows_done % w.B: rows_done % w.B + 32]
        t0 = time.perf_counter()
        O.sample_workload(O.REF, w, nthreads=1, rows=sel)
        t_total += time.perf_counter() - t0
        rows_done += len(sel)
    us_per_row = t_total / rows_done * 1e6
    # all host cores, rows spread over threads (reported beside it)
    nth = os.cpu_count() or 1
    nth = min(nth, 16)
    t0 = time.perf_counter()
    O.sample_workload(O.REF, w, nthreads=nth)
    t_all = time.perf_counter() - t0
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": 1e6 / us_per_row,
        "unit": "tokens/s",
        "cores": 1,
        "cpu_model": model,
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"{rows_done} rows of the {w.name} workload (oracle ref mode, 1 thread, "
                  f"{t_total:.1f} s); us/row {us_per_row:.0f}",
        "all_cores": {"threads": nth, "tokens_per_s": w.B / t_all, "step_ms": t_all * 1e3},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sets", type=int, default=0, help="logit copies rotated (0 = auto)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the short runs of the other configs")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES, 10 times (the "
                         "reference kernel for scaling HBM traffic counters)")
    ap.add_argument("--cpu-configs", action="store_true",
                    help="only time the CPU baseline (oracle ref mode) on a bounded sample of "
                         "every config and print one JSON line (no GPU)")
    ap.add_argument("--mask-probe", choices=["top_k", "top_p"], default=None,
                    help="only time one mask form (apply_top_k at C3's shape, apply_top_p at "
                         "C4's) and print its line")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only: rows are independent, so N GPUs "
              "each sample B/N rows with no communication; run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.cpu_configs:
        from llmk import synth
        out = {}
        for name in ("C1", "C2", "C3", "C4", "C5"):
            w = synth.make(name)
            out[name] = cpu_baseline(w, budget_s=4.0)
            log(f"[bench] cpu {name}: {out[name]}")
        print(json.dumps(out), flush=True)
        return
    import numpy as np
    import torch
    if args.copy_probe:
        n = args.copy_probe // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": 4 * n, "copies": 10}), flush=True)
        return
    import llmk
    from llmk import synth
    if args.mask_probe:
        print(json.dumps(time_mask(llmk, synth, torch, args.mask_probe)), flush=True)
        return
    w = synth.make(args.config)
    dev = torch.device("cuda:0")
    db0 = w.to_device(dev)
    step_bytes = w.algorithmic_bytes()
    logit_bytes = db0.logits.numel() * db0.logits.element_size()
    dbs = rotated_sets(llmk, db0, logit_bytes, args.sets)
    nsets = len(dbs)
    s = llmk.HipSampler(max_batch=w.B, max_vocab=w.V)
    B = w.B
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    cnt = torch.empty(B, dtype=torch.int32, device=dev)
    prepared = [s.prepare(d, tok, out_count=cnt) for d in dbs]
    stream = torch.cuda.current_stream()

    back_to_back(torch, s, prepared, args.warmup, stream)
    K = args.steps
    # timed steps: K back-to-back launches between two events on the launch
    # stream; the time per step is also the stream kernel's average duration
    # (one call per step, nothing between calls)
    ms_per_step = back_to_back(torch, s, prepared, K, stream)
    value = B / (ms_per_step * 1e-3)
    achieved = step_bytes / (ms_per_step * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic(args.config)
    log(f"[bench] {w.name}: {ms_per_step*1e3:.2f} us/step, {achieved:.0f} GB/s algorithmic, "
        f"sets {nsets}; traffic {traffic} ({traffic_src})")

    read_gbps = stream_read_gbps(torch)
    log(f"[bench] streaming read probe (2 GiB): {read_gbps:.0f} GB/s")
    others = None
    if not args.no_other_configs:
        others = {}
        for name in ("C1", "C2", "C3", "C4", "C5", "C3-f16", "C3-counts", "C5-counts",
                     "C3-seed1001"):
            if name == args.config:
                continue
            others[name] = time_config(llmk, synth, torch, name)
            log(f"[bench] {name}: {others[name]}")
        for op in ("top_k", "top_p"):
            others[f"apply_{op}"] = time_mask(llmk, synth, torch, op)
            log(f"[bench] apply_{op}: {others[f'apply_{op}']}")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w)
        log(f"[bench] cpu baseline: {cpu}")

    esz = "f32" if w.dtype == "f32" else "bf16"
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "us_per_step": ms_per_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": esz,
        "data": f"synthetic (seeded, {w.name} distributions); {nsets} logit copies rotated",
        "config": {
            "workload": f"{w.name}: B={w.B} V={w.V} {esz} logits, top-k 50, top-p 0.95, T 0.7, "
                        "repetition 1.1 / presence 0.5 / frequency 0.3, histories 2048 Zipf(1.1)"
                        if w.name == "C3" else w.name,
            "batch": w.B, "vocab": w.V, "algorithmic_bytes_per_step": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": "llmk::stream_kernel + llmk::xs_kernel (one call)",
            "kernel_avg_us": ms_per_step * 1e3,
            "achievable_read_GBps": read_gbps,
            "frac_of_achievable": achieved / read_gbps,
        },
        "other_configs": others,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
