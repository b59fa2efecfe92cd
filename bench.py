"""Benchmark of the token-sampling hot path on one MI355X.

Default workload (BASELINE.json's metric): the extended pipeline -- repetition/presence/frequency penalties over dense
int32 counts, a u32 grammar bitmask, temperature, top-k 50 / top-p 0.9, fused max/log-sum-exp (log-probabilities on),
inverse-CDF draw from one uniform per row -- at B=256, V=151,936 fp32, inputs resident in HBM. One step = one
gbs_sample_rows launch over the batch. Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--workload northstar|c1|c2|c3|c4|c5|keyed|markov] [--no-cpu]
                    [--no-per-config]

The default run (north star) also measures configs 1-5 and the keyed (reference-parity) sampler, each with its own CPU
baseline, and reports them under "per_config" in the same line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "sampled rows/sec + achieved HBM GB/s at B=256, V=151936 fp32, 1 MI355X"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="northstar")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--per-config-steps", type=int, default=100)
    ap.add_argument("--per-config-cpu-seconds", type=float, default=3.0)
    ap.add_argument("--no-per-config", action="store_true", help="north star only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 316,026,880 bytes device to device (the plain copy that scales rocprofv3 FETCH_SIZE)")
    return ap.parse_args()


def algorithmic_bytes(rows, vocab, logit_bytes, counts, mask, extra=0):
    per_row = logit_bytes * vocab + (4 * vocab if counts else 0) + (4 * ((vocab + 31) // 32) if mask else 0)
    return rows * per_row + extra


def profiled_traffic(workload):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE + WRITE_SIZE (scaled by a plain copy of known size), as
    recorded in profiles/; None when no measurement of this workload is recorded."""
    import re
    path = os.path.join(ROOT, "profiles", {"northstar": "sample_fast_k_northstar.md", "keyed": "keyed_fast_k_b256.md",
                                           "c5": "spec_verify_config5.md", "c3": "fs_split_kernels_config3.md"}.get(workload, ""))
    if not os.path.isfile(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", open(path).read())
    return int(m.group(1)) if m else None


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def copies_for(nbytes):
    """Input copies the timed launches rotate over: enough that the copies together are twice the Infinity Cache, so
    every launch reads inputs that earlier launches have pushed out of it (at most 16)."""
    return max(1, min(16, -(-2 * MALL_BYTES // max(nbytes, 1))))


def time_launches(launch, steps, warmup):
    import torch
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        launch()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def host_threads():
    """(threads used, cores this process may run on): every core the box gives the process, capped at 16, the CPU share
    of one GPU on this pool."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16)), n


def cpu_baseline_sample(cfg, seconds, threads):
    """The oracle's extended pipeline (the build's CPU restatement, there is no reference code for it) over the same
    batch, repeated until `seconds` of wall time have passed."""
    import numpy as np

    from oracle import oracle as O
    x = cfg["logits"]
    dt = O.DTYPE_BF16 if cfg["dtype"] == "bf16" else O.DTYPE_F32
    rows = x.shape[0]
    done, t0 = 0, time.perf_counter()
    while True:
        O.sample_rows(x, dt, cfg["counts"], cfg["mask"], cfg["params"], cfg["uniforms"], threads=threads)
        done += rows
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return done / el, done, el


def measure(wl, args, steps, cpu_seconds, dev, lib, stream):
    """Times `steps` launches of workload `wl` after `args.warmup` untimed ones; returns its record (and the CPU
    baseline over `cpu_seconds` unless --no-cpu)."""
    import numpy as np
    import torch

    from rexl3_amd import sampling as S
    from rexl3_amd import workloads as W

    threads, ncores = host_threads()
    cores_note = f"{threads} threads of the {ncores} cores this process may use (capped at 16, one GPU's CPU share)"
    cpu = None
    if wl in ("northstar", "c1", "c2", "c3", "c4", "mixed"):
        cfg = {"northstar": W.northstar, "c1": W.config1, "c2": W.config2, "c3": W.config3, "c4": W.config4,
               "mixed": W.northstar}[wl]()
        kmax = 0 if wl == "c3" else 64
        if wl == "mixed":
            # an engine's decode round: every tenth row samples top-p over the whole vocabulary (top_k 0)
            cfg["params"]["top_k"][::10] = 0
            kmax = -1  # GBS_KMAX_MIXED
        x = cfg["logits"]
        rows, vocab = x.shape
        is_bf16 = cfg["dtype"] == "bf16"
        nbytes = algorithmic_bytes(rows, vocab, 2 if is_bf16 else 4, cfg["counts"] is not None, cfg["mask"] is not None)
        ncopy = copies_for(nbytes)
        xts, cts, mts = [], [], []
        for _ in range(ncopy):
            xt = torch.from_numpy(x).to(dev)
            xts.append(xt.view(torch.bfloat16) if is_bf16 else xt)
            cts.append(None if cfg["counts"] is None else torch.from_numpy(cfg["counts"]).to(dev))
            mts.append(None if cfg["mask"] is None else torch.from_numpy(cfg["mask"]).to(dev))
        xt, ct, mt = xts[0], cts[0], mts[0]
        pt = torch.from_numpy(np.ascontiguousarray(cfg["params"]).view(np.uint8)).to(dev)
        ut = torch.from_numpy(cfg["uniforms"]).to(dev)
        out = {k: torch.empty(rows, dtype=torch.int32 if k in ("ids", "greedy", "status") else torch.float32, device=dev)
               for k in ("ids", "greedy", "status", "probs", "logprobs")}
        wsb = lib.gbs_sample_workspace_bytes(rows, vocab, kmax)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        lib.gbs_workspace_clear(ws.data_ptr(), wsb, stream)
        P = lambda t: None if t is None else C.c_void_p(t.data_ptr())  # noqa: E731
        # log-probabilities are part of the north star's pipeline (its log-softmax); configs 1-4 ask for the token, its
        # probability and the greedy id only
        want_lp = wl in ("northstar", "mixed")
        outputs = "ids, greedy, status, probs" + (", logprobs" if want_lp else "")
        argvs = [(P(xts[i]), 1 if is_bf16 else 0, rows, vocab, vocab, P(cts[i]), P(mts[i]), P(pt), P(ut), kmax, P(out["ids"]),
                  P(out["greedy"]), P(out["probs"]), P(out["logprobs"]) if want_lp else None, P(out["status"]), P(ws), wsb, stream)
                 for i in range(ncopy)]
        fn = lib.gbs_sample_rows
        turn = [0]

        def launch():
            rc = fn(*argvs[turn[0] % ncopy])
            turn[0] += 1
            if rc:
                raise RuntimeError(f"gbs_sample_rows returned {rc}")

        ms = time_launches(launch, steps, args.warmup)
        # the full path (kmax 0) runs split over fs_* launches when there are fewer rows than CUs
        kernel = ("fs_pass0_k + fs_hist_k + fs_collect_k" if rows < 256 else "sample_full_k") if kmax == 0 else "sample_fast_k"
        if kmax < 0:
            kernel = "sample_fast_k + fs_hist_k + fs_collect_k over the rows it leaves over"
        dtype = "bf16->f32" if is_bf16 else "f32"
        workload = {"northstar": "extended pipeline: penalties (dense i32 counts) + u32 grammar mask + T 0.8 + top-k 50 / top-p 0.9"
                                 " + log-softmax + inverse-CDF draw",
                    "c1": "config 1: single row, T 0.7, top-k 50, top-p 0.9",
                    "c2": "config 2: bf16 batched, per-row T, top-k 40, top-p 0.95, min-p 0.05",
                    "c3": "config 3: penalties over dense counts, T 0.8, top-p 0.9 over the whole vocabulary (no top-k)",
                    "c4": "config 4: grammar mask, top-k 64, top-p 0.95",
                    "mixed": "north-star batch with every tenth row at top_k 0 (top-p over the whole vocabulary), per-row "
                             "dispatch (GBS_KMAX_MIXED)"}[wl]
        st = out["status"].cpu().numpy()
        assert (st[cfg["params"]["temperature"] >= 0] >= 0).all()
        if not args.no_cpu:
            v, done, el = cpu_baseline_sample(cfg, cpu_seconds, threads)
            sub = min(rows, 8)
            v1, done1, el1 = cpu_baseline_sample({**cfg, "logits": cfg["logits"][:sub], "counts": None if cfg["counts"] is None
                                                  else cfg["counts"][:sub], "mask": None if cfg["mask"] is None else cfg["mask"][:sub],
                                                  "params": cfg["params"][:sub], "uniforms": cfg["uniforms"][:sub]},
                                                 min(2.0, cpu_seconds), 1)
            cpu = {"value": round(v, 1), "unit": "rows/s", "cores": threads, "host_cores": ncores, "kind": "port",
                   "sample": f"the build's C oracle of the same pipeline on the same {rows}-row batch, repeated for "
                             f"{el:.1f} s ({done} rows) on {cores_note}; 1 thread: {v1:.1f} rows/s ({done1} rows)",
                   "gbps": round(algorithmic_bytes(1, vocab, 2 if is_bf16 else 4, ct is not None, mt is not None) * v / 1e9, 3)}
    elif wl == "keyed":
        # the reference-parity keyed sampler: top-(k+8) of full f32 rows + try_choose, B=256, V=151,936
        cfg = W.northstar()
        x = cfg["logits"]
        rows, vocab = x.shape
        ncopy = copies_for(algorithmic_bytes(rows, vocab, 4, False, False))
        xts = [torch.from_numpy(x).to(dev) for _ in range(ncopy)]
        recs = S.keyed_rows([S.Sampling(seed=11, temperature=0.8, top_k=50, top_p=0.9, min_p=0.0)] * rows, list(range(rows)))
        pt = torch.from_numpy(recs.view(np.uint8)).to(dev)
        oi = torch.empty(rows, dtype=torch.int32, device=dev)
        os_ = torch.empty(rows, dtype=torch.int32, device=dev)
        wsb = lib.gbs_keyed_sample_workspace_bytes(rows, vocab)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        lib.gbs_workspace_clear(ws.data_ptr(), wsb, stream)
        argvs = [(C.c_void_p(xts[i].data_ptr()), 0, rows, vocab, vocab, C.c_void_p(pt.data_ptr()), 0, C.c_void_p(oi.data_ptr()), None,
                  C.c_void_p(os_.data_ptr()), C.c_void_p(ws.data_ptr()), wsb, stream) for i in range(ncopy)]
        fn = lib.gbs_keyed_sample_rows
        turn = [0]

        def launch():
            rc = fn(*argvs[turn[0] % ncopy])
            turn[0] += 1
            if rc:
                raise RuntimeError(f"gbs_keyed_sample_rows returned {rc}")

        ms = time_launches(launch, steps, args.warmup)
        nbytes = algorithmic_bytes(rows, vocab, 4, False, False)
        kernel = "keyed_fast_k"
        dtype = "f32 (choose in f64)"
        workload = "keyed sampler (reference parity): exact top-58 of full rows + try_choose (T 0.8, top-k 50, top-p 0.9)"
        if not args.no_cpu:
            from oracle import oracle as O
            t0 = time.perf_counter()
            done = 0
            while time.perf_counter() - t0 < cpu_seconds:
                O.batch_keyed_sample(x, O.DTYPE_F32, vocab, recs, 0, threads=threads)
                done += rows
            el = time.perf_counter() - t0
            cpu = {"value": round(done / el, 1), "unit": "rows/s", "cores": threads, "host_cores": ncores, "kind": "port",
                   "sample": f"C restatement of the reference CPU path (try_top_candidates(row, 58) + try_choose) on the same "
                             f"batch, {done} rows in {el:.1f} s on {cores_note}"}
    elif wl == "c5":
        cfg = W.config5()
        n_seq, width = cfg["n_seq"], cfg["width"]
        R, vocab = cfg["target"].shape
        ncopy = copies_for(2 * R * vocab * 4)
        tts = [torch.from_numpy(cfg["target"]).to(dev) for _ in range(ncopy)]
        dts = [torch.from_numpy(cfg["draft"]).to(dev) for _ in range(ncopy)]
        di = torch.from_numpy(cfg["draft_ids"]).to(dev)
        te = torch.from_numpy(cfg["temperatures"]).to(dev)
        ua = torch.from_numpy(cfg["u_accept"]).to(dev)
        ur = torch.from_numpy(cfg["u_resample"]).to(dev)
        acc = torch.empty(n_seq, dtype=torch.int32, device=dev)
        toks = torch.empty((n_seq, width + 1), dtype=torch.int32, device=dev)
        stt = torch.empty(n_seq, dtype=torch.int32, device=dev)
        wsb = lib.gbs_spec_verify_workspace_bytes(n_seq, width, vocab)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        lib.gbs_workspace_clear(ws.data_ptr(), wsb, stream)
        P = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
        argvs = [(P(tts[i]), P(dts[i]), n_seq, width, vocab, vocab, P(di), P(te), P(ua), P(ur), P(acc), P(toks), P(stt), P(ws), wsb,
                  stream)
                 for i in range(ncopy)]
        fn = lib.gbs_spec_verify
        turn = [0]

        def launch():
            rc = fn(*argvs[turn[0] % ncopy])
            turn[0] += 1
            if rc:
                raise RuntimeError(f"gbs_spec_verify returned {rc}")

        ms = time_launches(launch, steps, args.warmup)
        rows = R
        nbytes = 2 * R * vocab * 4
        kernel = ("spec_rows_k" if R >= 192 else "spec_split_k") + " + spec_exact_k + spec_draw_k"
        dtype = "f32 (integer masses)"
        workload = "config 5: speculative verification, 32 sequences x (7 drafts + 1 bonus), rejection + residual resampling"
        if not args.no_cpu:
            from oracle import oracle as O
            t0 = time.perf_counter()
            done = 0
            while time.perf_counter() - t0 < cpu_seconds:
                O.spec_verify(cfg["target"], cfg["draft"], n_seq, width, cfg["draft_ids"], cfg["temperatures"], cfg["u_accept"],
                              cfg["u_resample"], threads=threads)
                done += R
            el = time.perf_counter() - t0
            cpu = {"value": round(done / el, 1), "unit": "rows/s", "cores": threads, "host_cores": ncores, "kind": "port",
                   "sample": f"the build's C oracle of the same verification on the same batch (its sequences over the "
                             f"threads), {done} rows in {el:.1f} s on {cores_note}"}
    elif wl == "markov":
        # the DSV4 draft head's keyed Markov walk: 8 walk rows over V = 129,280 (bf16 embed / head [V, 256])
        walk_rows, vocab = 8, 129_280
        rng = np.random.default_rng(8)
        x = (rng.standard_normal((walk_rows, vocab)) * 2).astype(np.float32)
        tab = lambda: torch.from_numpy(((rng.standard_normal((vocab, 256)) * 0.1).astype(np.float32).view(np.uint32) >> 16)  # noqa: E731
                                       .astype(np.uint16).view(np.int16)).to(dev).view(torch.bfloat16)
        emb, hed = tab(), tab()
        lg = torch.from_numpy(x).to(dev)
        ids = torch.zeros(walk_rows + 1, dtype=torch.int32, device=dev)
        ids[0] = 17
        cand = torch.empty((walk_rows, 1024), dtype=torch.int32, device=dev)
        scores = torch.empty(1024, dtype=torch.float32, device=dev)
        conf = torch.empty(walk_rows, dtype=torch.float32, device=dev)
        P = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
        fn = lib.gb_dsv4_mtp_markov_walk_keyed_bf16
        argv = (P(lg), P(ids), P(conf), P(emb), P(hed), P(cand), P(scores), walk_rows, vocab, 256, 16, 1234, 0.8, 0.9, 0.0, 100,
                stream)

        def launch():
            rc = fn(*argv)
            if rc:
                raise RuntimeError(f"gb_dsv4_mtp_markov_walk_keyed_bf16 returned {rc}")

        ms = time_launches(launch, steps, args.warmup)
        rows = walk_rows
        # the logits once (candidates), then per row 1024 head rows and one embedding row of 512 B
        nbytes = walk_rows * vocab * 4 + walk_rows * (1024 + 1) * 512
        kernel = "mw_cands_k + 8 x (mw_bias_k + mw_pick_k<true>)"
        dtype = "f32 bias from bf16 tables (choose in f64)"
        workload = "DSV4 draft head's keyed Markov walk: 8 walk rows, V 129,280, rank 256, top-16 keyed choose (launch-bound)"
        if not args.no_cpu:
            from oracle import oracle as O
            eb = (emb.view(torch.int16).cpu().numpy()).view(np.uint16)
            hb = (hed.view(torch.int16).cpu().numpy()).view(np.uint16)
            t0 = time.perf_counter()
            done = 0
            while time.perf_counter() - t0 < min(cpu_seconds, 10.0):
                O.markov_walk(x, 17, eb, hb, walk_rows, True, 16, 1234, 0.8, 0.9, 0.0, 100)
                done += walk_rows
            el = time.perf_counter() - t0
            cpu = {"value": round(done / el, 1), "unit": "walk rows/s", "cores": 1, "host_cores": ncores, "kind": "port",
                   "sample": f"the build's C oracle of the same walk (one thread), {done} walk rows in {el:.1f} s"}
    else:
        raise SystemExit(f"unknown workload {wl}")
    achieved = nbytes / (ms / 1e3) / 1e9
    ncopy = locals().get("ncopy", 1)
    outputs = locals().get("outputs")
    return dict(name=wl, workload=workload, kernel=kernel, dtype=dtype, rows=rows, vocab=vocab, steps=steps, ms=ms, copies=ncopy,
                rows_per_s=rows / (ms / 1e3), bytes=nbytes, achieved=achieved, cpu=cpu, outputs=outputs)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box in this run has one, and the sampler shards by rows with no "
              f"communication. --gpus {args.gpus} is not supported.", file=sys.stderr)
        sys.exit(2)
    import torch

    from rexl3_amd import _lib

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(316_026_880 // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "launches": 3}))
        return
    lib = _lib.load()
    stream = C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    r = measure(args.workload, args, args.steps, args.cpu_seconds, dev, lib, stream)
    per_config = None
    if args.workload == "northstar" and not args.no_per_config:
        per_config = {}
        for wl in ("c1", "c2", "c3", "c4", "c5", "keyed", "mixed"):
            print(f"# per-config {wl}", file=sys.stderr, flush=True)
            q = measure(wl, args, args.per_config_steps, args.per_config_cpu_seconds, dev, lib, stream)
            per_config[wl] = {"workload": q["workload"], "kernel": q["kernel"], "rows": q["rows"], "vocab": q["vocab"],
                              "input_copies": q["copies"], **({"outputs": q["outputs"]} if q["outputs"] else {}),
                              "steps": q["steps"], "ms_per_step": round(q["ms"], 5), "rows_per_s": round(q["rows_per_s"], 1),
                              "bytes_per_launch": q["bytes"], "achieved_gbps": round(q["achieved"], 1),
                              "frac": round(q["achieved"] / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(wl),
                              "cpu_baseline": q["cpu"]}
            torch.cuda.empty_cache()
    line = {
        "metric": METRIC,
        "value": round(r["rows_per_s"], 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": r["dtype"],
        "data": "synthetic: seeded splitmix64 logits (Box-Muller normals + peaks), Zipf(1.1) 4096-token count histories, "
                "log-uniform grammar masks; resident in HBM before timing, the timed launches rotating over input copies "
                "twice the 256 MB Infinity Cache in size",
        "config": {"workload": r["workload"], "name": r["name"], "rows": r["rows"], "vocab": r["vocab"], "kernel": r["kernel"],
                   "input_copies": r["copies"]},
        "hbm_gbps": round(r["achieved"], 1),
        "roofline": {"bound": "hbm", "achieved": round(r["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["achieved"] / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(r["name"]),
                     "bytes_per_launch": r["bytes"], "timing": "HIP events around the timed launches on their stream"},
        "cpu_baseline": r["cpu"],
    }
    if per_config is not None:
        line["per_config"] = per_config
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
