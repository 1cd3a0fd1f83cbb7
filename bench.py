"""Benchmark: the full N=1 decode matvec set of the 36-layer trunk plus the
tied Q8_0 output head, on one MI355X.

Workload (synthetic, seeded, random-init weights of the real shapes):
  per layer, VQ dim 4, nc 4096, 2 residual stages, DQV3, bf16 activations:
    q 4096x2560, k 1024x2560, v 1024x2560, head gate 16x2560   (one launch, shared x)
    o 2560x4096                                                 (one launch)
    gate 10240x2560, up 10240x2560                              (one launch, shared x)
    down 2560x10240                                             (one launch)
  head: Q8_0 151936x2560 (one launch)
A step is one token: the 145 launches in forward order on one stream,
replayed as one HIP graph (native plan, sparkmv_plan_*). Weights and inputs
are resident in HBM before timing starts.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--mode graph|eager]
                    [--workload decode-set|ffn-up|q6k-down|verify8|prefill512|forward|verify-block|
                                decode-set-q6k|prompt512|decode-chain|startup]

Prints one JSON line (rank 0). The metric is time per token (lower is
better); achieved GB/s over the algorithmic bytes (container + bf16 x + f32 y
per matvec) and the VQ kernel's roofline fraction come with it, plus the
oracle's CPU time for a bounded sample of the same set.
"""
import argparse
import concurrent.futures
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "spark-x2.6-4b-q6k_amd"))

PEAK_GBPS = 8000.0
PEAK_F16_TFLOPS = 2500.0

LAYERS, HIDDEN, FFN, QD, KVD, NHEAD = 36, 2560, 10240, 4096, 1024, 16
VOCAB = 151936
VQ = dict(dim=4, nc=4096, nstages=2, v3=1)
METRIC = "decode matvec µs/token (36-layer trunk, N=1) + achieved HBM GB/s vs peak"

# per layer: (name, rows, cols, launch group)
LAYER_MATS = [("q", QD, HIDDEN, 0), ("k", KVD, HIDDEN, 0), ("v", KVD, HIDDEN, 0), ("g", NHEAD, HIDDEN, 0),
              ("o", HIDDEN, QD, 1), ("gate", FFN, HIDDEN, 2), ("up", FFN, HIDDEN, 2), ("down", HIDDEN, FFN, 3)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def seed_of(layer, idx):
    return 0x5EED0000 + 97 * layer + idx


def gen_layer(sm, layer):
    return [sm.synth_container(seed_of(layer, i), r, c, VQ["dim"], VQ["nc"], VQ["nstages"], VQ["v3"])
            for i, (_, r, c, _) in enumerate(LAYER_MATS)]


def algorithmic_bytes_vq(nbytes_container, rows, cols, ncol=1):
    """Container bytes + bf16 x + f32 y of one matvec."""
    return nbytes_container + 2 * cols * ncol + 4 * rows * ncol


class DecodeSet:
    """The per-token decode matvec set as recorded: the plan, every op's
    output tensor, the shared inputs, and (for the layers asked for) the
    host containers, so the outputs can be checked after timing."""

    def __init__(self):
        self.plan = None
        self.op_bytes = None
        self.op_kind = []
        self.hosts = {}      # layer -> list of container bytes (LAYER_MATS order), for kept layers
        self.ys = {}         # layer -> list of (matrix index, y tensor [ncol, >= rows])
        self.xs = {}         # cols -> (device bf16 [ncol, cols], host f32 [ncol, cols])
        self.head = None     # host Q8_0 blocks
        self.head_rows = 0
        self.logits = None
        self.ncol = 1


def build_decode_set(sm, torch, dev, ncol=1, head_rows=VOCAB, layers=LAYERS, keep_hosts=()):
    """Generate, upload and record the per-token chain. Returns a DecodeSet;
    the host containers of the layers in keep_hosts stay in it."""
    ds = DecodeSet()
    ds.ncol, ds.head_rows = ncol, head_rows
    t0 = time.time()
    with concurrent.futures.ThreadPoolExecutor(min(16, os.cpu_count() or 4)) as ex:
        hosts = list(ex.map(lambda l: gen_layer(sm, l), range(layers)))
        head_future = ex.submit(sm.synth_q8_0, 0x4EAD, head_rows, HIDDEN)
        head = head_future.result()
    log(f"generated {layers} layers + head in {time.time() - t0:.1f} s")
    for c in (HIDDEN, QD, FFN):
        xb = sm.synth_bf16(c, ncol * c)
        ds.xs[c] = (torch.from_numpy(xb.view(np.int16).reshape(ncol, c).copy()).to(dev),
                    sm.bf16_to_f32(xb).reshape(ncol, c))
    xs = {c: v[0] for c, v in ds.xs.items()}
    plan = sm.Plan()
    op_bytes, op_kind = [], []
    devs = []
    for l in range(layers):
        mats = [sm.DeviceContainer(h, dev) for h in hosts[l]]
        devs.append(mats)
        ys = [torch.zeros(ncol, r, device=dev) for (_, r, _, _) in LAYER_MATS]
        for grp in range(4):
            idx = [i for i, m in enumerate(LAYER_MATS) if m[3] == grp]
            cols = LAYER_MATS[idx[0]][2]
            if len(set(LAYER_MATS[i][1] for i in idx)) > 1 and ncol > 1:
                # one ldy per launch: give every matrix of the group a buffer of the widest row count
                w = max(LAYER_MATS[i][1] for i in idx)
                for i in idx:
                    ys[i] = torch.zeros(ncol, w, device=dev)
            plan.add_vq([mats[i] for i in idx], xs[cols], [ys[i] for i in idx], ncols=ncol, accumulate=False,
                        label=f"L{l}:" + "+".join(LAYER_MATS[i][0] for i in idx))
            op_bytes.append(sum(algorithmic_bytes_vq(hosts[l][i].nbytes, LAYER_MATS[i][1], cols, ncol) for i in idx))
            op_kind.append("vq")
        ds.ys[l] = list(enumerate(ys))
        if l in keep_hosts:
            ds.hosts[l] = hosts[l]
        hosts[l] = None
    hb = torch.from_numpy(head).to(dev)
    logits = torch.zeros(ncol, head_rows, device=dev)
    plan.add_kquant("q8_0", hb, head_rows, HIDDEN, xs[HIDDEN], logits, ncols=ncol, label="head")
    op_bytes.append(head.nbytes + 2 * HIDDEN * ncol + 4 * head_rows * ncol)
    op_kind.append("q8_0")
    plan.keep.append((devs, hb, logits, xs))
    torch.cuda.synchronize()
    log(f"uploaded in {time.time() - t0:.1f} s total")
    ds.plan, ds.op_bytes, ds.op_kind = plan, np.array(op_bytes, dtype=np.float64), op_kind
    ds.head, ds.logits = head, logits
    return ds


def check_decode_set(ds, layers):
    """The output check (oracle, after timing): each kept layer's outputs against
    the oracle's bit-exact decode times x in f64, every row and column, and
    every head row against the closed-form Q8_0 dot. Returns the largest
    relative L2 error per launch group."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import chain_check as cc
    return cc.check_decode_set(ds, LAYER_MATS, layers)


def bench_decode_set_q6k(args, sm, torch, dev):
    """The same 36-layer N=1 chain with the trunk as ggml Q6_K blocks (the
    GGUF's trunk, one k-quant launch per matrix) and the tied Q8_0 head."""
    stream = torch.cuda.Stream(device=dev)
    t0 = time.time()
    with torch.cuda.stream(stream):
        xb = {c: sm.synth_bf16(c, c) for c in (HIDDEN, QD, FFN)}
        xs = {c: torch.from_numpy(xb[c].view(np.int16).reshape(1, c).copy()).to(dev) for c in (HIDDEN, QD, FFN)}
        plan = sm.Plan()
        op_bytes = []
        kept = (0, LAYERS // 2, LAYERS - 1)
        groups = []   # kept layers' (key, host blocks, rows, cols, y) for the output check
        with concurrent.futures.ThreadPoolExecutor(min(16, os.cpu_count() or 4)) as ex:
            futs = [[ex.submit(sm.synth_q6k, seed_of(l, i), r, c) for i, (_, r, c, _) in enumerate(LAYER_MATS)]
                    for l in range(LAYERS)]
            head = sm.synth_q8_0(0x4EAD, args.head_rows, HIDDEN)
            for l in range(LAYERS):
                # the matrices that share x are stacked by rows into one launch
                # (q, k, v, head gate; gate, up), as the reference's own fused
                # qkv tensor is (model.rs:44-55): rows are independent, so each
                # row's result is the one a separate launch gives
                for grp in range(4):
                    idx = [i for i, m in enumerate(LAYER_MATS) if m[3] == grp]
                    c = LAYER_MATS[idx[0]][2]
                    r = sum(LAYER_MATS[i][1] for i in idx)
                    blocks = np.concatenate([futs[l][i].result() for i in idx])
                    d = torch.from_numpy(blocks).to(dev)
                    y = torch.zeros(r, device=dev)
                    key = "+".join(LAYER_MATS[i][0] for i in idx)
                    plan.add_kquant("q6_k", d, r, c, xs[c], y, label=f"L{l}:" + key)
                    plan.keep.append((d, y))
                    if l in kept:
                        groups.append((key, blocks, r, c, y))
                    op_bytes.append(blocks.nbytes + 2 * c + 4 * r)
                futs[l] = None
        hb = torch.from_numpy(head).to(dev)
        logits = torch.zeros(args.head_rows, device=dev)
        plan.add_kquant("q8_0", hb, args.head_rows, HIDDEN, xs[HIDDEN], logits, label="head")
        plan.keep.append((hb, logits, xs))
        op_bytes.append(head.nbytes + 2 * HIDDEN + 4 * args.head_rows)
        torch.cuda.synchronize()
        log(f"generated and uploaded the Q6_K trunk in {time.time() - t0:.1f} s")
        ms = time_steps(plan, torch, stream, args.steps, args.warmup, args.mode)
        op_ms = plan.time_ops(stream, iters=max(3, min(args.steps, 10)))
    op_bytes = np.array(op_bytes, dtype=np.float64)
    total = float(op_bytes.sum())
    trunk_b, trunk_ms = float(op_bytes[:-1].sum()), float(op_ms[:-1].sum())
    log(f"  step {ms * 1e3:.1f} us ({args.mode}); Q6_K kernels {trunk_ms * 1e3:.1f} us over {len(op_ms) - 1} launches "
        f"({trunk_b / (trunk_ms * 1e-3) / 1e9:.1f} GB/s); head {op_ms[-1] * 1e3:.1f} us")
    achieved = trunk_b / (trunk_ms * 1e-3) / 1e9
    check = None
    if args.check:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import chain_check as cc
        t = time.time()
        res = cc.check_kquant_set(groups, {c: sm.bf16_to_f32(v) for c, v in xb.items()}, head, args.head_rows, logits)
        log(f"  output check ({time.time() - t:.1f} s): {res}")
        check = {"rel_l2_max": max(res.values()), "detail": res, "layers": list(kept),
                 "method": "every row of the kept layers' launches vs the oracle's Q6_K dequant times x in f64; "
                           "every head row vs the closed-form Q8_0 dot"}
    return {
        "metric": "decode matvec us/token (36-layer Q6_K trunk, N=1, tied Q8_0 head)",
        "value": round(ms * 1e3, 2), "unit": "us/token", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 dot2 -> f32 (bf16 x)", "data": "synthetic (seeded, random-init Q6_K blocks of the real shapes)",
        "config": {"workload": "36-layer N=1 decode matvec set, Q6_K trunk + Q8_0 head", "layers": LAYERS,
                   "hidden": HIDDEN, "ffn": FFN, "launches_per_step": len(op_ms), "mode": args.mode},
        "achieved_gbps": round(total / (ms * 1e-3) / 1e9, 1),
        "frac_of_peak": round(total / (ms * 1e-3) / 1e9 / PEAK_GBPS, 4),
        "algorithmic_bytes_per_step": int(total),
        "roofline": {"bound": "hbm", "kernel": "q6k_gemv_staged_kernel", "achieved": round(achieved, 1),
                     "peak": PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4), "traffic": None},
        "check": check,
    }


def time_steps(plan, torch, stream, steps, warmup, mode):
    if mode == "graph":
        plan.run(stream)                  # one-time launch setup outside the capture
        torch.cuda.synchronize()
        plan.capture(stream)
    run = plan.launch if mode == "graph" else plan.run
    for _ in range(warmup):
        run(stream)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        run(stream)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def cpu_baseline_decode_set(sample_layers=LAYERS, head_rows=VOCAB, reps=9):
    """The oracle's runtime path (model.rs:209-234): containers decoded to f32
    once, then a row-parallel 8-lane dot per matvec, all host threads. By
    default the whole token is timed (every layer and the full head, one
    layer decoded at a time, the median of `reps` runs of each); a smaller
    sample is scaled to one token."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import sparkmv as sm
    import sparkref as ref
    nth = ref.threads()
    per_layer = []
    for l in range(sample_layers):
        hosts = gen_layer(sm, l)
        Ws = [ref.decode(h) for h in hosts]
        xs = {c: sm.bf16_to_f32(sm.synth_bf16(c, c)) for c in (HIDDEN, QD, FFN)}
        best = []
        for _ in range(reps):
            t = time.perf_counter()
            for (_, r, c, _), W in zip(LAYER_MATS, Ws):
                ref.matvec(W, xs[c], nth)
            best.append(time.perf_counter() - t)
        per_layer.append(np.median(best))
        del Ws
    blocks = sm.synth_q8_0(0x4EAD, head_rows, HIDDEN)
    Wh = ref.q8_0_dequant(blocks, head_rows, HIDDEN)
    xh = sm.bf16_to_f32(sm.synth_bf16(HIDDEN, HIDDEN))
    th = []
    for _ in range(reps):
        t = time.perf_counter()
        ref.matvec(Wh, xh, nth)
        th.append(time.perf_counter() - t)
    us = (np.mean(per_layer) * LAYERS + np.median(th) * VOCAB / head_rows) * 1e6
    whole = sample_layers == LAYERS and head_rows == VOCAB
    return {"value": round(float(us), 1), "unit": "us/token", "cores": int(nth), "kind": "port",
            "sample": f"oracle decode-to-f32 + row-parallel 8-lane dot (model.rs:209-234) on {sample_layers} of "
                      f"{LAYERS} layers and {head_rows} of {VOCAB} head rows, median of {reps} per layer and for the "
                      f"head" + (", summed: one whole token" if whole else ", scaled to one token")}


def bench_decode_set(args, sm, torch, dev):
    stream = torch.cuda.Stream(device=dev)
    ncol = 8 if args.workload == "verify8" else 1
    check_layers = (0, LAYERS // 2, LAYERS - 1) if args.check else ()
    with torch.cuda.stream(stream):
        ds = build_decode_set(sm, torch, dev, ncol=ncol, head_rows=args.head_rows, keep_hosts=check_layers)
        plan, op_bytes, op_kind = ds.plan, ds.op_bytes, ds.op_kind
        ms = time_steps(plan, torch, stream, args.steps, args.warmup, args.mode)
        op_ms = plan.time_ops(stream, iters=max(3, min(args.steps, 10)))
        torch.cuda.synchronize()
    total_bytes = float(op_bytes.sum())
    vq = np.array([k == "vq" for k in op_kind])
    vq_bytes, vq_ms = float(op_bytes[vq].sum()), float(op_ms[vq].sum())
    n_vq = int(vq.sum())
    achieved = vq_bytes / (vq_ms * 1e-3) / 1e9
    head_ms = float(op_ms[~vq].sum())
    groups = {}
    for lab, b, t in zip(plan.labels, op_bytes, op_ms):
        key = lab.split(":")[-1]
        g = groups.setdefault(key, [0.0, 0.0, 0])
        g[0] += b
        g[1] += t
        g[2] += 1
    per_group = {}
    for k, (b, t, n) in groups.items():
        log(f"  {k:16s} {n:3d} launches  {t / n * 1e3:8.2f} us/kernel  {b / (t * 1e-3) / 1e9:8.1f} GB/s")
        per_group[k] = {"launches": n, "kernel_us": round(t / n * 1e3, 3), "bytes_per_launch": int(b / n),
                        "gbps": round(b / (t * 1e-3) / 1e9, 1)}
    log(f"  step {ms * 1e3:.1f} us ({args.mode}); sum of kernel times {op_ms.sum() * 1e3:.1f} us")
    workload = ("36-layer N=8 verify matvec set (trunk + Q8_0 head), weights decoded once per step"
                if ncol == 8 else "36-layer N=1 decode matvec set + tied Q8_0 head")
    out = {
        "metric": METRIC,
        "value": round(ms * 1e3, 2),
        "unit": "us/token" if ncol == 1 else "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16xf16->f32 (bf16 x)",
        "data": "synthetic (seeded, random-init weights of the real shapes)",
        "config": {"workload": workload, "layers": LAYERS, "hidden": HIDDEN, "ffn": FFN, "q_dim": QD, "kv_dim": KVD,
                   "vq": "dim 4, nc 4096, 2 stages, DQV3 12-bit", "head": f"Q8_0 {args.head_rows}x{HIDDEN}",
                   "columns": ncol, "launches_per_step": len(op_ms), "mode": args.mode},
        "achieved_gbps": round(total_bytes / (ms * 1e-3) / 1e9, 1),
        "frac_of_peak": round(total_bytes / (ms * 1e-3) / 1e9 / PEAK_GBPS, 4),
        "algorithmic_bytes_per_step": int(total_bytes),
        "roofline": {"bound": "hbm", "kernel": "vq_mfma_kernel", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": recorded_traffic(ncol),
                     "bytes_per_launch": round(vq_bytes / n_vq), "avg_launch_us": round(vq_ms / n_vq * 1e3, 3),
                     "timing": "kernel-exact: start/stop events carried by each dispatch (hipExtLaunchKernel) on the "
                               "launch stream, averaged over eager runs of the plan",
                     "per_group": per_group,
                     "head_q8_0": {"us": round(head_ms * 1e3, 2),
                                   "gbps": round(float(op_bytes[~vq].sum()) / (head_ms * 1e-3) / 1e9, 1)}},
    }
    if check_layers:
        t = time.time()
        res = check_decode_set(ds, check_layers)
        log(f"  output check ({time.time() - t:.1f} s): " + ", ".join(f"{k} {v:.2e}" for k, v in res.items()))
        out["check"] = {"rel_l2_max": max(res.values()), "per_group": {k: float(f"{v:.3e}") for k, v in res.items()},
                        "layers": list(check_layers), "head_rows": args.head_rows, "columns": ncol,
                        "method": "outputs of the timed plan vs the oracle's decode x f64 (all rows of the layers "
                                  "listed, every head row)"}
    return out


def bench_decode_chain(args, sm, torch, dev):
    """decode-chain: the 36-layer N=1 matvec chain with every op depending on
    the one before it, as in the forward (q+k+v+g from rms_norm(h), o from q,
    gate+up from rms_norm(h + o), down from gelu(gate) * up into the residual),
    as ONE persistent launch (sparkmv_chain_*), then the Q8_0 head; the
    dataflow of sparkmv.DecodeChain."""
    t0 = time.time()
    with concurrent.futures.ThreadPoolExecutor(min(16, os.cpu_count() or 4)) as ex:
        hosts = list(ex.map(lambda l: gen_layer(sm, l), range(LAYERS)))
        head = sm.synth_q8_0(0x4EAD, args.head_rows, HIDDEN)
    layers = [{n: sm.DeviceContainer(h, dev) for (n, _, _, _), h in zip(LAYER_MATS, hl)} for hl in hosts]
    nbytes = sum(h.nbytes for hl in hosts for h in hl) + head.nbytes
    kept = (0, LAYERS // 2, LAYERS - 1)
    hosts = {l: {n: h for (n, _, _, _), h in zip(LAYER_MATS, hosts[l])} for l in kept}
    log(f"generated and uploaded in {time.time() - t0:.1f} s")
    h0 = torch.from_numpy(sm.bf16_to_f32(sm.synth_bf16(0xE0, HIDDEN))).to(dev)
    dc = sm.DecodeChain(layers, torch.from_numpy(head).to(dev), args.head_rows, h0)
    dc.chain.tune(args.chain_waves, args.chain_look, args.chain_units)
    stream = torch.cuda.Stream(device=dev)
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            dc.launch(stream)
        torch.cuda.synchronize()
        dc.chain.status()
        a, b = ev(), ev()
        a.record(stream)
        for _ in range(args.steps):
            dc.launch(stream)
        b.record(stream)
        torch.cuda.synchronize()
        dc.chain.status()
        ms = a.elapsed_time(b) / args.steps
        c0, c1 = ev(), ev()
        c0.record(stream)
        for _ in range(args.steps):
            dc.chain.launch(stream)
        c1.record(stream)
        torch.cuda.synchronize()
        dc.chain.status()
        chain_ms = c0.elapsed_time(c1) / args.steps
    log(f"  decode chain: {ms * 1e3:.1f} us/token ({chain_ms * 1e3:.1f} us for the chain launch), "
        f"{nbytes / (ms * 1e-3) / 1e9:.0f} GB/s of weights")
    phases = None
    if args.chain_trace:
        buf = dc.chain.trace(True, device=dev)
        with torch.cuda.stream(stream):
            dc.chain.launch(stream)
        torch.cuda.synchronize()
        dc.chain.status()
        dc.chain.trace(False)
        tr = buf.cpu().numpy()
        if args.chain_trace_out:
            np.save(args.chain_trace_out, tr)
        phases = chain_phases(tr, dc.chain.labels)
        for k, v in phases.items():
            log(f"  phases {k}: " + ", ".join(f"{a} {b}" for a, b in v.items()))
    out = {"metric": "decode matvec us/token, dependent chain (36-layer trunk as one persistent launch + Q8_0 head)",
           "value": round(ms * 1e3, 2), "unit": "us/token", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
           "vs_baseline": None, "dtype": "f16xf16->f32 (bf16 x), f64 norm sums",
           "data": "synthetic (seeded, random-init weights of the real shapes)",
           "config": {"workload": "decode chain: 144 dependent VQ matvecs with rms_norm/gelu staging, one launch, "
                                  "then the Q8_0 head", "layers": LAYERS, "hidden": HIDDEN, "ffn": FFN,
                      "head": f"Q8_0 {args.head_rows}x{HIDDEN}", "waves": args.chain_waves,
                      "look": args.chain_look, "min_units": args.chain_units},
           "chain_launch_us": round(chain_ms * 1e3, 2), "weight_bytes": int(nbytes), "phases_us": phases,
           "achieved_gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
           "frac_of_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_GBPS, 4)}
    if args.check:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import chain_check as cc
        t = time.time()
        res = cc.check_decode_chain(dc, hosts, head, kept)
        log(f"  output check ({time.time() - t:.1f} s): {res}")
        out["check"] = {"rel_l2_max": cc.worst_matvec(res), "detail": res, "layers": list(kept),
                        "method": "each op of the timed chain vs the oracle from the inputs the GPU read; every "
                                  "head row"}
    return out


def chain_phases(tr, labels):
    """Per op kind (the label after the layer prefix), medians over the
    layers of the median workgroup's phases: req (op start to x requested),
    spin (x requested to x arrived everywhere), stage (to x staged), enter
    (to the step loop's start), loop (wave 0's steps), tail (to every unit
    done), epi (to the stores issued); handoff (the op before's last
    workgroup's stores to this op's median x arrival) and span (last stores
    of the op before to last stores of this one). tr: [workgroups, ops, 8]
    clock ticks of 10 ns, then the shader clock at each op's start and end
    (their ratio to the 100 MHz clock gives the shader clock's rate)."""
    clk = tr[:, :, 8:].astype(np.int64)
    t = tr[:, :, :8].astype(np.int64)
    t = (t - t[0, 0, 0] + (1 << 31)) % (1 << 32) - (1 << 31)   # signed ticks from workgroup 0's start
    t = t * 0.01   # us
    dt = t[:, :, 6] - t[:, :, 0]
    ok = dt > 0.5
    ghz = float(np.median(((clk[:, :, 1] - clk[:, :, 0]) % (1 << 32))[ok] / (dt[ok] * 1e3)))
    kinds = {}
    for i, lab in enumerate(labels):
        kinds.setdefault(lab.split(":", 1)[-1], []).append(i)
    names = ("req", "spin", "stage", "enter", "loop", "tail", "epi", "handoff", "span")
    out = {}
    for k, idx in kinds.items():
        rows = []
        for i in idx:
            if i == 0:
                continue
            a = t[:, i]
            last_prev = t[:, i - 1, 6].max()
            md = lambda u, v: np.median(a[:, v] - a[:, u])  # noqa: E731
            rows.append([md(0, 7), md(7, 1), md(1, 2), md(2, 3), md(3, 4), md(4, 5), md(5, 6),
                         np.median(a[:, 1]) - last_prev, a[:, 6].max() - last_prev])
        if rows:
            m = np.median(np.array(rows), axis=0)
            out[k] = {n: round(float(v), 2) for n, v in zip(names, m)}
    out["shader_clock_ghz"] = {"median": round(ghz, 3)}
    return out


FW_WINDOW = 512   # sliding_window; 9 of the 36 layers are full attention (every fourth)


def bench_forward(args, sm, torch, dev):
    """The whole decode token on the GPU (sparkmv_model_forward): embedding
    row, 36 layers of norm / qkv + head gate / rope + KV store / attention /
    out / norm / gate + up / gelu / down, final norm, Q8_0 tied head. The
    cache is first filled with `context` tokens (untimed); then each step is
    one token at the next position, replayed as one HIP graph."""
    prompt = args.workload == "prompt512"
    P = 0 if prompt else args.context
    max_ctx = (512 if prompt else P + args.warmup + args.steps) + 16
    cfg = dict(hidden=HIDDEN, layers=LAYERS, heads=NHEAD, kv_heads=KVD // (QD // NHEAD), head_dim=QD // NHEAD,
               intermediate=FFN, vocab=args.head_rows, eps=1e-6, sliding_window=FW_WINDOW, rope_full_theta=5.0e6,
               rope_full_partial=0.25, rope_slide_theta=1.0e4, rope_slide_partial=1.0, max_ctx=max_ctx,
               x_dtype=sm.X_F32 if args.fw_x == "f32" else sm.X_BF16, dim=VQ["dim"], nc=VQ["nc"],
               nstages=VQ["nstages"], v3=VQ["v3"])
    xdesc = "f32 x (the reference's precision: hi + lo f16 halves)" if args.fw_x == "f32" else "bf16 x"
    shapes = [("qkv", QD + 2 * KVD, HIDDEN), ("attn_gate", NHEAD, HIDDEN), ("out", HIDDEN, QD),
              ("gate", FFN, HIDDEN), ("up", FFN, HIDDEN), ("down", HIDDEN, FFN)]
    t0 = time.time()
    rng = np.random.default_rng(5)

    def gen(l):
        return [sm.synth_container(seed_of(l, 20 + i), r, c, VQ["dim"], VQ["nc"], VQ["nstages"], VQ["v3"])
                for i, (_, r, c) in enumerate(shapes)]

    layers, mat_bytes = [], 0
    with concurrent.futures.ThreadPoolExecutor(min(16, os.cpu_count() or 4)) as ex:
        futs = [ex.submit(gen, l) for l in range(LAYERS)]
        head = sm.synth_q8_0(0x4EAD, args.head_rows, HIDDEN)
        for l, f in enumerate(futs):
            hosts = f.result()
            L = {name: sm.DeviceContainer(h, dev) for (name, _, _), h in zip(shapes, hosts)}
            mat_bytes += sum(h.nbytes for h in hosts)
            for name in ("in_norm", "post_norm"):
                L[name] = torch.from_numpy((1 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32)).to(dev)
            L["full"] = l % 4 == 3
            layers.append(L)
    norm = torch.from_numpy((1 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32)).to(dev)
    model = sm.Model(cfg, layers, torch.from_numpy(head).to(dev), norm)
    log(f"generated and uploaded the model in {time.time() - t0:.1f} s")
    stream = torch.cuda.Stream(device=dev)
    logits = torch.zeros(args.head_rows, device=dev)
    toks = np.random.default_rng(6).integers(0, args.head_rows, size=max_ctx)
    ev = lambda: torch.cuda.Event(enable_timing=True)
    if prompt:
        hd = torch.from_numpy(head).to(dev)
        make_f32 = lambda: sm.Model(dict(cfg, x_dtype=sm.X_F32), layers, hd, norm)  # noqa: E731  same weights
        return bench_prompt(args, model, stream, logits, toks, mat_bytes, head, ev, torch, make_f32)
    with torch.cuda.stream(stream):
        t0 = time.time()
        for p in range(P):
            model.forward(int(toks[p]), p, logits, stream)
        torch.cuda.synchronize()
        log(f"filled {P} positions of the cache in {time.time() - t0:.1f} s")
        a, b = ev(), ev()
        a.record(stream)
        for p in range(P, P + 4):
            model.forward(int(toks[p]), p, logits, stream)
        b.record(stream)
        torch.cuda.synchronize()
        eager_us = a.elapsed_time(b) / 4 * 1e3
        if args.workload == "verify-block":
            # a block of 8 drafted tokens at position P + 4, rolled back after each step
            blk = torch.zeros((8, args.head_rows), device=dev)
            P4 = P + 4
            for _ in range(args.warmup):
                model.verify([int(t) for t in toks[P4:P4 + 8]], P4, blk, stream)
                model.rollback(P4)
            torch.cuda.synchronize()
            a, b = ev(), ev()
            a.record(stream)
            for _ in range(args.steps):
                model.verify([int(t) for t in toks[P4:P4 + 8]], P4, blk, stream)
                model.rollback(P4)
            b.record(stream)
            torch.cuda.synchronize()
            vms = a.elapsed_time(b) / args.steps
            log(f"  verify block of 8: {vms * 1e3:.1f} us (eager), {vms * 1e3 / 8:.1f} us per token; "
                f"single token {eager_us:.1f} us eager")
            return {
                "metric": "speculative verify block us/step (8 tokens, whole model, tied Q8_0 head)",
                "value": round(vms * 1e3, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
                "warmup": args.warmup, "ms_per_step": round(vms, 4), "higher_is_better": False, "scaling": "weak",
                "vs_baseline": None, "dtype": f"f16xf16->f32 matvecs ({xdesc}), f32 elementwise, f64 norm sums",
                "data": "synthetic (seeded, random-init weights of the real shapes)",
                "config": {"workload": f"verify block of 8 tokens at context {P4}", "layers": LAYERS,
                           "hidden": HIDDEN, "ffn": FFN, "heads": NHEAD, "sliding_window": FW_WINDOW,
                           "head": f"Q8_0 {args.head_rows}x{HIDDEN}", "mode": "eager"},
                "single_token_eager_us": round(eager_us, 1),
            }
        model.capture(logits, stream)
        pos = P + 4
        for _ in range(args.warmup):
            model.replay(int(toks[pos]), pos, stream)
            pos += 1
        torch.cuda.synchronize()
        a, b = ev(), ev()
        a.record(stream)
        for _ in range(args.steps):
            model.replay(int(toks[pos]), pos, stream)
            pos += 1
        b.record(stream)
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    assert bool(torch.isfinite(logits).all()), "non-finite logits"
    kvd = KVD
    n_full = sum(1 for L in layers if L["full"])
    mid = P + 4 + args.warmup + args.steps // 2
    kv_bytes = (n_full * mid + (LAYERS - n_full) * min(FW_WINDOW, mid)) * kvd * 4 * 2
    total = mat_bytes + head.nbytes + kv_bytes
    log(f"  step {ms * 1e3:.1f} us (graph), {eager_us:.1f} us eager; context {P}; "
        f"{total / (ms * 1e-3) / 1e9:.1f} GB/s over weights + KV")
    return {
        "metric": "decode forward us/token (whole model: embedding, 36 layers, tied Q8_0 head)",
        "value": round(ms * 1e3, 2),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"f16xf16->f32 matvecs ({xdesc}), f32 elementwise, f64 norm sums",
        "data": "synthetic (seeded, random-init weights of the real shapes)",
        "config": {"workload": "decode forward, one token per step at context " + str(P), "layers": LAYERS,
                   "hidden": HIDDEN, "ffn": FFN, "heads": NHEAD, "kv_heads": cfg["kv_heads"],
                   "head_dim": cfg["head_dim"], "sliding_window": FW_WINDOW, "full_layers": n_full,
                   "vq": "dim 4, nc 4096, 2 stages, DQV3 12-bit", "head": f"Q8_0 {args.head_rows}x{HIDDEN}",
                   "mode": "graph (token and position in device memory)"},
        "eager_us_per_token": round(eager_us, 1),
        "bytes_per_token": int(total),
        "achieved_gbps": round(total / (ms * 1e-3) / 1e9, 1),
        "frac_of_peak": round(total / (ms * 1e-3) / 1e9 / PEAK_GBPS, 4),
    }


def bench_prompt(args, model, stream, logits, toks, mat_bytes, head, ev, torch, make_f32=None):
    """prompt512: one 512-token prompt chunk through the whole model
    (sparkmv_model_forward_batch, the reference's forward_batch + tail_logits,
    vq-model-gpu.cu:858-953, over the 512-token chunks of :1161-1173): every
    matvec on the prefill GEMM over the chunk's tokens, batched norms, rope +
    KV store and causal attention, then the last token's final norm and head.
    Each step runs the chunk at position 0 and rolls the cache back."""
    N = 512
    chunk = [int(t) for t in toks[:N]]
    model.reserve(N)
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            model.forward_batch(chunk, 0, logits, stream)
            model.rollback(0)
        torch.cuda.synchronize()
        a, b = ev(), ev()
        a.record(stream)
        for _ in range(args.steps):
            model.forward_batch(chunk, 0, logits, stream)
            model.rollback(0)
        b.record(stream)
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    assert bool(torch.isfinite(logits).all()), "non-finite logits"
    check = None
    if args.check:
        # The same 512 tokens one decode step at a time (the decode path,
        # which the tests hold to the oracle), with bf16 activations as the
        # chunk has and, on a second model over the same weights, with f32
        # ones. The f32/bf16 gap is what bf16 activations alone move the
        # logits by at this depth; the chunk (f16 x and folded stages in its
        # GEMMs, besides bf16 activations) is held to twice that gap.
        prompt_logits = logits.clone()
        t = time.time()

        def decode_logits(m):
            out = torch.empty_like(logits)
            m.rollback(0)
            with torch.cuda.stream(stream):
                for p, tok in enumerate(chunk):
                    m.forward(tok, p, out, stream)
            torch.cuda.synchronize()
            m.rollback(0)
            return out.double()

        def rl2(a, b):
            return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))

        dec16 = decode_logits(model)
        m32 = make_f32()
        m32.reserve(N)
        dec32 = decode_logits(m32)
        del m32
        g = prompt_logits.double()
        err, gap, err32 = rl2(g, dec16), rl2(dec16, dec32), rl2(g, dec32)
        agree = int(torch.argmax(g)) == int(torch.argmax(dec16)) == int(torch.argmax(dec32))
        log(f"  check ({time.time() - t:.1f} s): last logits vs 512 bf16 decode steps relL2 {err:.2e} "
            f"(vs f32 decode steps {err32:.2e}; f32 vs bf16 decode {gap:.2e}), argmax agrees {agree}")
        check = {"rel_l2_vs_bf16_decode": err, "rel_l2_vs_f32_decode": err32, "f32_vs_bf16_decode": gap,
                 "argmax_agrees": agree,
                 "method": "the chunk's last logits vs the same 512 tokens one decode step at a time "
                           "(sparkmv_model_forward, which the tests hold to the oracle), bf16 activations; bar: "
                           "twice the gap between the decode path's f32 and bf16 activations, argmax equal"}
        assert err <= 2 * max(gap, 1e-3) and agree, f"prompt chunk vs the decode path: {check}"
    # matvec work: 2 flop per weight and token over the trunk, the head for one token
    weights = LAYERS * ((QD + 2 * KVD + NHEAD) * HIDDEN + HIDDEN * QD + 3 * FFN * HIDDEN)
    flop = 2.0 * weights * N + 2.0 * args.head_rows * HIDDEN
    log(f"  prompt chunk of {N}: {ms * 1e3:.1f} us, {N / (ms * 1e-3):.0f} tokens/s, "
        f"{flop / (ms * 1e-3) / 1e12:.0f} TFLOP/s of matvec work")
    return {
        "metric": "prompt chunk us/chunk (512 tokens at position 0, whole model, last token's logits)",
        "value": round(ms * 1e3, 2), "unit": "us/chunk", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16xf16->f32 prefill GEMM (bf16 x rounded to f16), f32 elementwise",
        "data": "synthetic (seeded, random-init weights of the real shapes)",
        "config": {"workload": "prompt chunk of 512 tokens at position 0", "layers": LAYERS, "hidden": HIDDEN,
                   "ffn": FFN, "heads": NHEAD, "sliding_window": FW_WINDOW, "head": f"Q8_0 {args.head_rows}x{HIDDEN}",
                   "mode": "eager"},
        "tokens_per_s": round(N / (ms * 1e-3), 1),
        "matvec_tflops": round(flop / (ms * 1e-3) / 1e12, 1),
        "weight_bytes": int(mat_bytes + head.nbytes),
        "check": check,
    }


def recorded_traffic(ncol):
    """HBM bytes per VQ launch measured by rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE in separate runs, each scaled by the same counter's reading
    for a copy of known size); the summary file under profiles/ says how."""
    path = os.path.join(ROOT, "profiles", "traffic_decode-set.json")
    if ncol != 1 or not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    return rec.get("vq_bytes_per_launch")


def copy_calibration(torch, dev, mib):
    """A plain device copy of `mib` MiB (read mib, write mib), run a few
    times so a counter run sees a kernel of known traffic."""
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"copy calibration: {mib} MiB copied 3 times")


def bench_single(args, sm, torch, dev):
    """ffn-up: one VQ GEMV 10240x2560 (N=1); q6k-down: one Q6_K GEMV
    2560x10240. A step is one call; the plan holds COPIES distinct copies of
    the matrix (more bytes than the 256 MB memory-side cache) called back to
    back in one graph, so each call reads cold weights without host launch
    cost, and the step time is the graph time over the copies."""
    copies = 16
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        plan = sm.Plan()
        if args.workload == "ffn-up":
            x = torch.from_numpy(sm.synth_bf16(2, HIDDEN).view(np.int16).reshape(1, HIDDEN).copy()).to(dev)
            y = torch.zeros(1, FFN, device=dev)
            data = sm.synth_container(1, FFN, HIDDEN)
            for _ in range(copies):
                m = sm.DeviceContainer(data, dev)
                plan.add_vq([m], x, [y])
                plan.keep.append(m)
            nbytes = algorithmic_bytes_vq(data.nbytes, FFN, HIDDEN)
            kernel = "vq_mfma_kernel"
        elif args.workload == "q6k-down":
            host = sm.synth_q6k(3, HIDDEN, FFN)
            x = torch.from_numpy(sm.synth_bf16(4, FFN).view(np.int16).reshape(1, FFN).copy()).to(dev)
            y = torch.zeros(1, HIDDEN, device=dev)
            for _ in range(copies):
                blocks = torch.from_numpy(host).to(dev)
                plan.add_kquant("q6_k", blocks, HIDDEN, FFN, x, y)
                plan.keep.append(blocks)
            nbytes = host.nbytes + 2 * FFN + 4 * HIDDEN
            kernel = "q6k_gemv_staged_kernel"
        else:
            raise SystemExit(f"unknown workload {args.workload}")
        plan.keep.append((x, y))
        torch.cuda.synchronize()
        ms = time_steps(plan, torch, stream, args.steps, args.warmup, args.mode) / copies
        op_ms = plan.time_ops(stream, iters=5)
    kern = float(np.mean(op_ms))
    gbps = nbytes / (ms * 1e-3) / 1e9
    kgbps = nbytes / (kern * 1e-3) / 1e9
    log(f"  {args.workload}: {ms * 1e3:.2f} us/call back to back, kernel {kern * 1e3:.2f} us, {kgbps:.0f} GB/s")
    shape = "VQ 10240x2560 (dim 4, nc 4096, 2 stages)" if args.workload == "ffn-up" else "Q6_K 2560x10240"
    return {"metric": f"single GEMV us/call, {shape}, N=1, bf16 x", "value": round(ms * 1e3, 3), "unit": "us/call",
            "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16xf16->f32 (bf16 x)", "data": "synthetic",
            "config": {"workload": args.workload, "copies_in_graph": copies}, "achieved_gbps": round(gbps, 1),
            "frac_of_peak": round(gbps / PEAK_GBPS, 4), "algorithmic_bytes_per_step": int(nbytes),
            "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(kgbps, 1), "peak": PEAK_GBPS,
                         "unit": "GB/s", "frac": round(kgbps / PEAK_GBPS, 4), "traffic": None,
                         "bytes_per_launch": int(nbytes), "avg_launch_us": round(kern * 1e3, 3)}}


def bench_startup(args, sm, torch, dev):
    """startup: what one launch's fixed cost is made of, on the hot kernel's
    launch shape (sparkmv_probe_startup): an empty kernel, the 64 KB codebook
    staging alone, and plain reads of 8, 20 and 40 MB (about o, down and
    gate+up) cold, with address translation warm (one dword per 4 KB page
    read just before) and with the data warm (one dword per 64-byte line);
    then the decode set's 145 launches as plain reads of their byte counts in
    one graph (sparkmv_probe_read_chain), and what a dependent op costs
    inside one launch instead (sparkmv_probe_handoff), three ways."""
    sizes = (8 << 20, 20 << 20, 40 << 20)
    res = sm.probe_startup(sizes, reps=max(5, min(args.steps, 64)))
    out = {"empty_kernel_us": round(res["empty"], 2), "empty_kernel_1wave_us": round(res["empty_1wave"], 2),
           "empty_kernel_1wg_us": round(res["empty_1wg"], 2),
           "empty_back_to_back_stream_us": round(res["empty_stream"], 2),
           "empty_back_to_back_graph_us": round(res["empty_graph"], 2),
           "stage_64k_us": round(res["stage_64k"], 2), "reads": {}}
    for b in sizes:
        r = res[b]
        mb = b >> 20
        out["reads"][f"{mb}MB"] = {k: round(v, 2) for k, v in r.items()}
        out["reads"][f"{mb}MB"]["cold_gbps"] = round(b / (r["cold"] * 1e-6) / 1e9, 1)
        log(f"  read {mb} MB: cold {r['cold']:.2f} us ({b / (r['cold'] * 1e-6) / 1e9:.0f} GB/s), translation warm "
            f"{r['page_warm']:.2f} us, data warm {r['line_warm']:.2f} us")
    # the decode set's 145 launches as plain reads of the same byte counts
    # (one layer's containers give every layer's sizes), back to back in one
    # graph: the floor of one launch per matvec with no compute
    hosts = gen_layer(sm, 0)
    layer = []
    for grp in range(4):
        idx = [i for i, m in enumerate(LAYER_MATS) if m[3] == grp]
        layer.append(sum(algorithmic_bytes_vq(hosts[i].nbytes, LAYER_MATS[i][1], LAYER_MATS[i][2]) for i in idx))
    head = VOCAB * (HIDDEN // 32) * 34 + 2 * HIDDEN + 4 * VOCAB
    chain = layer * LAYERS + [head]
    rc = sm.probe_read_chain(chain, reps=max(5, min(args.steps, 64)))
    out["read_chain"] = {"launches": len(chain), "bytes": int(sum(chain)), "per_layer_bytes": layer, "head_bytes": head,
                         "graph_us": round(rc["graph_us"], 1), "stream_us": round(rc["stream_us"], 1),
                         "graph_gbps": round(sum(chain) / (rc["graph_us"] * 1e-6) / 1e9, 1)}
    log(f"  the decode set's {len(chain)} launches as plain reads ({sum(chain) / 1e9:.3f} GB): "
        f"{rc['graph_us']:.1f} us per graph replay, {rc['stream_us']:.1f} us eager")
    hand = sm.probe_handoff((1280, 2560, 5120))
    out["handoff_us_per_op"] = {k: {str(n): round(v, 2) for n, v in d.items()} for k, d in hand.items()}
    for k, d in hand.items():
        log(f"  dependent handoff, {k}: " + ", ".join(f"{n} words {v:.2f} us" for n, v in d.items()))
    log(f"  empty kernel {res['empty']:.2f} us ({res['empty_1wave']:.2f} with one wave per workgroup, "
        f"{res['empty_1wg']:.2f} with one workgroup), 64 KB codebook staging {res['stage_64k']:.2f} us; "
        f"back to back per launch: {res['empty_stream']:.2f} us on a stream, {res['empty_graph']:.2f} us in a graph")
    return {"metric": "launch start-up split: kernel-exact us per launch on the hot kernel's shape",
            "value": out["reads"]["20MB"]["cold"], "unit": "us (20 MB cold read)", "n_gpus": 1, "steps": args.steps,
            "warmup": 0, "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "u32 reads",
            "data": "synthetic", "config": {"workload": "startup", "grid": "one workgroup of 10 waves per CU",
                                            "sizes_MB": [b >> 20 for b in sizes]},
            "startup": out}


def bench_prefill(args, sm, torch, dev):
    """prefill512: the prompt GEMM of one FFN pair, W 10240x2560 (up) and
    2560x10240 (down), VQ dim 4 nc 4096 2 stages, against 512 bf16 tokens.
    A step is both GEMMs; MFMA-bound, so the roofline is TFLOP/s."""
    ntok = 512
    stream = torch.cuda.Stream(device=dev)
    mats = []
    with torch.cuda.stream(stream):
        for i, (r, c) in enumerate(((FFN, HIDDEN), (HIDDEN, FFN))):
            m = sm.DeviceContainer(sm.synth_container(0x9F00 + i, r, c), dev)
            x = torch.from_numpy(sm.synth_bf16(0x9F10 + i, ntok * c).view(np.int16).reshape(ntok, c).copy()).to(dev)
            y = torch.zeros(ntok, r, device=dev)
            mats.append((m, x, y, r, c))
        torch.cuda.synchronize()

        def step():
            for m, x, y, _, _ in mats:
                m.prefill(x, y, stream=stream)

        def timed():
            for _ in range(args.warmup):
                step()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                step()
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / args.steps
        # the default: the two stages folded into one f16 weight; then the
        # same step with each stage's exact codewords accumulated apart
        assert sm.prefill_fold()
        ms = timed()
        with sm.prefill_mode(False):
            ms_apart = timed()
        # the same step through the reference's ABI: xT [cols][ntok] f32, one
        # launch per stage, tiled variant 2 with the runtime's 128 x 64 tile
        # (vq-model-gpu.cu:296-299, :838-851); the null stream, as it uses
        L = sm.lib()
        xts = [x.float().t().contiguous() for _, x, _, _, _ in mats]
        torch.cuda.synchronize()

        def step_ref():
            for (m, _, y, r, c), xT in zip(mats, xts):
                for p in m.stage_ptrs:
                    sm.check(L.vqg_prefill_launch_tile(p, 4, 4096, r, c, 1, xT.data_ptr(), ntok, y.data_ptr(),
                                                       128, 64, 2), "reference-layout prefill")
        for _ in range(args.warmup):
            step_ref()
        torch.cuda.synchronize()
        r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        r0.record(torch.cuda.default_stream(dev))
        for _ in range(args.steps):
            step_ref()
        r1.record(torch.cuda.default_stream(dev))
        torch.cuda.synchronize()
        ms_ref = r0.elapsed_time(r1) / args.steps
    flops = sum(2.0 * ntok * r * c for _, _, _, r, c in mats)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"  reference ABI (xT f32, one launch per stage): {ms_ref * 1e3:.1f} us/step, "
        f"{flops / (ms_ref * 1e-3) / 1e12:.1f} TFLOP/s")
    nbytes = sum(m.host.data.nbytes + 2 * ntok * c + 4 * ntok * r for m, _, _, r, c in mats)
    log(f"  prefill {ntok} tokens, up + down: {ms * 1e3:.1f} us/step, {tflops:.1f} TFLOP/s (stages folded); "
        f"{ms_apart * 1e3:.1f} us/step, {flops / (ms_apart * 1e-3) / 1e12:.1f} TFLOP/s (stages apart)")
    return {"metric": "prefill GEMM us/step (N=512, FFN up + down)", "value": round(ms * 1e3, 2), "unit": "us/step",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16xf16->f32 (bf16 x)",
            "data": "synthetic (seeded, random-init weights of the real shapes)",
            "config": {"workload": "prefill GEMM, 512 bf16 tokens x (10240x2560 and 2560x10240 VQ)", "tokens": ntok,
                       "stages": "folded (g0 c0 + g1 c1 rounded to one f16 weight)"},
            "roofline": {"bound": "mfma", "kernel": "prefill_cw_kernel", "achieved": round(tflops, 1),
                         "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / PEAK_F16_TFLOPS, 4),
                         "traffic": None, "flops_per_step": flops, "bytes_per_step": int(nbytes)},
            "stages_apart": {"us_per_step": round(ms_apart * 1e3, 2),
                             "tflops": round(flops / (ms_apart * 1e-3) / 1e12, 1),
                             "mode": "sparkmv_prefill_fold(0): each stage's exact codewords, gains in f32"},
            "reference_abi": {"us_per_step": round(ms_ref * 1e3, 2),
                              "tflops": round(flops / (ms_ref * 1e-3) / 1e12, 1),
                              "route": "vqg_prefill_launch_tile variant 2, xT [cols][512] f32, one launch per stage"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mode", choices=["graph", "eager"], default="graph")
    ap.add_argument("--workload", default="decode-set",
                    choices=["decode-set", "verify8", "ffn-up", "q6k-down", "prefill512", "forward",
                             "verify-block", "decode-set-q6k", "decode-chain", "prompt512", "startup"])
    ap.add_argument("--context", type=int, default=1024, help="forward: positions cached before the timed steps")
    ap.add_argument("--head-rows", type=int, default=VOCAB)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--chain-waves", type=int, default=12, help="decode-chain: waves per workgroup")
    ap.add_argument("--chain-look", type=int, default=2, help="decode-chain: index steps in flight per wave")
    ap.add_argument("--chain-units", type=int, default=0,
                    help="decode-chain: units per workgroup aimed for (0: the chain's cost model)")
    ap.add_argument("--chain-trace", action="store_true", help="decode-chain: one more launch with a phase trace")
    ap.add_argument("--fw-x", choices=["bf16", "f32"], default="bf16",
                    help="forward / verify-block: the matvecs' activations (f32 is the reference's precision)")
    ap.add_argument("--chain-trace-out", default=None, metavar="NPY", help="decode-chain: also save the raw trace")
    ap.add_argument("--no-check", dest="check", action="store_false",
                    help="skip the oracle check of the timed outputs")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB on the device (for counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: the matvec path runs on a single MI355X, and multi-GPU "
                                   "sharding (by output rows, zero exchange) is described, not built",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import sparkmv as sm
    sm.lib()
    if not torch.cuda.is_available():
        sys.exit("no GPU visible")
    dev = torch.device("cuda:0")
    name = torch.cuda.get_device_name(0)
    log(f"device {name}")
    if args.calibrate_copy:
        copy_calibration(torch, dev, args.calibrate_copy)
    if args.workload in ("decode-set", "verify8"):
        out = bench_decode_set(args, sm, torch, dev)
        if not args.no_cpu_baseline and args.workload == "decode-set":
            t = time.time()
            out["cpu_baseline"] = cpu_baseline_decode_set()
            log(f"cpu baseline took {time.time() - t:.1f} s")
    elif args.workload == "prefill512":
        out = bench_prefill(args, sm, torch, dev)
    elif args.workload == "startup":
        out = bench_startup(args, sm, torch, dev)
    elif args.workload == "decode-set-q6k":
        out = bench_decode_set_q6k(args, sm, torch, dev)
    elif args.workload == "decode-chain":
        out = bench_decode_chain(args, sm, torch, dev)
    elif args.workload in ("forward", "verify-block", "prompt512"):
        out = bench_forward(args, sm, torch, dev)
    else:
        out = bench_single(args, sm, torch, dev)
    out["device"] = name
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
