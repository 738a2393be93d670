#!/usr/bin/env python3
"""Benchmark of the MI355X reduction + top-k path (one GPU).

A "step" is one pass of the hot path over one batch of the headline workload,
BASELINE configs[3] (the largest single-GPU config): a flat fp32 tensor of 2^28
N(0.5, 2) elements (1 GiB) reduced to a scalar six ways -- sum, mean, amax,
argmax, var and std (unbiased).  `value` is the step's algorithmic HBM bytes
(input read once + output written once, per op) divided by the step time: GB/s.

Inputs are resident in HBM before the timed region; consecutive ops rotate over
3 input buffers (3 GiB > the 256 MB Infinity Cache) so every op reads from HBM.
Times come from HIP events on the stream the kernels run on.  The other
BASELINE configs (C1 sum, C2 strided reductions, C3 topk, C5 logits topk /
argmax) are measured the same way and reported under "configs".

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline] [--vs-torch]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
# kernel each headline op launches (one launch per op: the split rows finish in the same launch)
DOMINANT_KERNEL = {"sum": "k_rows<SumOp,4,256,4>", "mean": "k_rows<SumOp,4,256,4>",
                   "amax": "k_rows<ArgOp<true>,4,256,4>", "argmax": "k_rows<ArgOp<true>,4,256,4>",
                   "var": "k_rows<WelfordOp,4,256,4>", "std": "k_rows<WelfordOp,4,256,4>"}
# the C2 strided ops
C2_KERNEL = {"mean_dim1": "k_cols<SumOp,4,64,4,512>",
             "amax_dim0": "k_cols<ArgOp<true>,4,256,2,256>", "argmax_dim0": "k_cols<ArgOp<true>,4,256,2,256>",
             "var_dim-1": "k_rows_reg_var<4,1,256>", "std_dim-1": "k_rows_reg_var<4,1,256>"}
METRIC = "achieved HBM GB/s (% of MI355X peak) for sum/argmax/topk; rows/s topk"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="headline workload only")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB copy (PMC calibration for FETCH/WRITE_SIZE)")
    ap.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles", "pmc_traffic.json"))
    ap.add_argument("--only", default="",
                    help="comma list of extra sections to run (default: all): " + ",".join(SECTIONS))
    ap.add_argument("--no-headline", action="store_true",
                    help="skip the headline step (profiling one section alone; `value` is then null)")
    ap.add_argument("--no-accuracy", action="store_true", help="skip the fp64 error report")
    ap.add_argument("--vs-torch", action="store_true",
                    help="also time PyTorch-ROCm's own kernels on the same shapes (reported under torch_rocm)")
    return ap.parse_args()


SECTIONS = ["C1", "C2", "C3", "C4f64", "C5", "softmax", "copy", "reduce_backward", "softmax_cols", "topk_short"]


class Call:
    """A pre-bound C-ABI launch (all argument marshalling done up front)."""

    def __init__(self, fn, args):
        self.fn, self.args = fn, args

    def __call__(self):
        rc = self.fn(*self.args)
        if rc != 0:
            from tensorplay_amd import _capi
            raise RuntimeError(_capi.lib().tpr_last_error().decode())


def reduce_call(torch, capi, x, op, dims, stream, correction=1):
    nd = x.dim()
    rd = sorted(set((d + nd) % nd for d in dims)) if dims is not None else list(range(nd))
    kept = [x.shape[i] for i in range(nd) if i not in rd]
    tmap = capi._torch_dtypes()
    idt = tmap[x.dtype]
    od = capi.default_out_dtype(op, idt)
    tdt = {v: k for k, v in tmap.items()}[od]
    out = torch.empty(kept, dtype=tdt, device=x.device)
    desc = capi.make_desc(op, list(x.shape), list(x.stride()), rd, od, correction, in_dtype=idt)
    L = capi.lib()
    wsb = L.tpr_reduce_workspace_bytes(ctypes.byref(desc))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    keep = (desc, out, ws)
    c = Call(L.tpr_reduce, (ctypes.byref(desc), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                            ctypes.c_void_p(ws.data_ptr()), wsb, stream))
    c.keep = keep
    c.out_bytes = out.numel() * out.element_size()
    return c


def topk_call(torch, capi, x, k, stream):
    rows, cols = x.shape
    dt = capi._torch_dtypes()[x.dtype]
    vals = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    idx = torch.empty((rows, k), dtype=torch.int64, device=x.device)
    L = capi.lib()
    wsb = L.tpr_topk_workspace_bytes(dt, rows, cols, k)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    c = Call(L.tpr_topk, (ctypes.c_void_p(x.data_ptr()), dt, rows, cols, x.stride(0), k, 1, 1,
                          ctypes.c_void_p(vals.data_ptr()), ctypes.c_void_p(idx.data_ptr()),
                          ctypes.c_void_p(ws.data_ptr()), wsb, stream))
    c.keep = (vals, idx, ws)
    c.out_bytes = rows * k * (x.element_size() + 8)
    return c


KIND_NAMES = {0: "k_copy_contig", 1: "k_copy_rows", 2: "k_copy_tile", 3: "k_copy_elem"}


def copy_kernel_name(plan):
    return KIND_NAMES[plan & 3] + ("_v" if plan & 2 == 2 and plan & 4 else "")


def copy_call(torch, capi, dst, src, stream):
    tmap = capi._torch_dtypes()
    desc = capi.make_copy_desc(list(dst.shape), list(dst.stride()), list(src.stride()), tmap[dst.dtype],
                               tmap[src.dtype])
    L = capi.lib()
    c = Call(L.tpr_copy, (ctypes.byref(desc), ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                          stream))
    c.keep = (desc, dst)
    c.bytes = src.numel() * src.element_size() + dst.numel() * dst.element_size()
    return c


def softmax_call(torch, capi, x, dim, mode, stream, y=None):
    """Pre-bound tpr_softmax on x (forward) or on g = x with output y (backward)."""
    v = capi._view3(x, dim)
    out = torch.empty(list(x.shape), dtype=torch.float32, device=x.device)
    d = capi.SoftmaxDesc()
    d.mode, d.dtype = mode, capi.FLOAT32
    d.outer, d.n, d.inner = v[0]
    vb = capi._view3(y, dim) if y is not None else None
    for k in range(3):
        d.a_strides[k] = v[1][k]
        d.b_strides[k] = vb[1][k] if vb is not None else 0
    L = capi.lib()
    wsb = L.tpr_softmax_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    c = Call(L.tpr_softmax, (ctypes.byref(d), ctypes.c_void_p(x.data_ptr()),
                             ctypes.c_void_p(y.data_ptr() if y is not None else 0),
                             ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb, stream))
    c.keep = (d, out, ws)
    c.bytes = x.numel() * 4 * (3 if y is not None else 2)
    return c


def nll_bwd_call(torch, capi, n, c, target, g, tw, stream):
    gi = torch.empty((n, c), dtype=torch.float32, device=target.device)
    call = Call(capi.lib().tpr_nll_loss_backward, (ctypes.c_void_p(g.data_ptr()), 1, ctypes.c_void_p(target.data_ptr()),
                                                   1, ctypes.c_void_p(0), ctypes.c_void_p(tw.data_ptr()), n, c, 1,
                                                   -100, ctypes.c_void_p(gi.data_ptr()), stream))
    call.keep = (gi,)
    call.bytes = n * c * 4 + n * 8
    return call


def reduce_bwd_call(torch, capi, x, op, dims, stream, g, res=None):
    nd = x.dim()
    rd = list(range(nd)) if dims is None else sorted(set((d + nd) % nd for d in dims))
    desc = capi.make_desc(op, list(x.shape), list(x.stride()), rd, capi.FLOAT32, 1)
    gi = torch.empty(list(x.shape), dtype=torch.float32, device=x.device)
    L = capi.lib()
    wsb = L.tpr_reduce_backward_workspace_bytes(ctypes.byref(desc))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    c = Call(L.tpr_reduce_backward, (ctypes.byref(desc), ctypes.c_void_p(g.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                     ctypes.c_void_p(res.data_ptr() if res is not None else 0),
                                     ctypes.c_void_p(gi.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb, stream))
    c.keep = (desc, gi, ws, g, res)
    # algorithmic bytes: write the gradient; var / std also read x once (the
    # least any implementation reads: the mean is not an input)
    c.bytes = x.numel() * 4 * (2 if op in ("var", "std") else 1)
    return c


def sample_call(torch, capi, x, k, temperature, top_p, u, stream):
    rows, cols = x.shape
    out = torch.empty((rows,), dtype=torch.int64, device=x.device)
    L = capi.lib()
    wsb = L.tpr_sample_workspace_bytes(capi.FLOAT32, rows, cols, k)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    c = Call(L.tpr_sample, (ctypes.c_void_p(x.data_ptr()), capi.FLOAT32, rows, cols, x.stride(0), k,
                            ctypes.c_float(temperature), ctypes.c_float(top_p), ctypes.c_void_p(u.data_ptr()),
                            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), wsb, stream))
    c.keep = (out, ws, u)
    c.bytes = x.numel() * 4 + rows * 12
    return c


def rate(ms, by):
    return {"ms": round(ms, 5), "GB/s": round(by / ms / 1e6, 1), "frac_of_peak": round(by / ms / 1e6 / HBM_PEAK_GBS, 4),
            "alg_bytes": by}


def time_calls(torch, step_fns, steps, warmup):
    """Run warmup, then time `steps` iterations of step_fns[i % len] with HIP events."""
    for i in range(warmup):
        step_fns[i % len(step_fns)]()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(steps):
        step_fns[i % len(step_fns)]()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps  # ms per iteration


def gen(torch, shape, kind, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    if kind == "normal":
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
    if kind == "uniform":
        return torch.rand(shape, generator=g, device=dev, dtype=torch.float32) * 2 - 1
    raise ValueError(kind)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the reduction/top-k path has no "
              "multi-GPU exchange); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from tensorplay_amd import _capi as capi

    capi.lib()  # fails loudly if the HIP library is not built
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    steps, warmup = args.steps, args.warmup
    only = set(x for x in args.only.split(",") if x) or set(SECTIONS)
    bad = only - set(SECTIONS)
    if bad:
        sys.exit(f"bench.py: unknown sections {sorted(bad)}; choose from {SECTIONS}")

    # ---------------- headline: configs[3] --------------------------------------
    n4 = 1 << 28
    nbuf = 3
    bufs = [gen(torch, (n4,), "normal", 4000 + i, dev) * 2.0 + 0.5 for i in range(nbuf)]
    in_bytes = n4 * 4
    ops4 = ["sum", "mean", "amax", "argmax", "var", "std"]
    calls = [[reduce_call(torch, capi, b, op, None, stream) for op in ops4] for b in bufs]
    op_bytes = [in_bytes + c.out_bytes for c in calls[0]]
    step_bytes = sum(op_bytes)
    result = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
              "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
              "data": "synthetic: torch.randn seeded on device, scaled to N(0.5, 2), 3 rotating 1 GiB buffers "
                      "(each op reads a different buffer than the op before it)",
              "config": {"workload": "configs[3]: flat fp32 tensor of 268,435,456 elements (1 GiB), N(0.5, 2); "
                                     "sum, mean, amax, argmax, var, std (unbiased) to a scalar. configs[3] is the "
                                     "largest single-GPU configuration; configs[0,1,2,4] are measured below under "
                                     "configs",
                         "step_alg_bytes": step_bytes}}
    step_fns = []

    if not args.no_headline:
        # Op j of step i reads buffer (6i + j) % 3, so consecutive ops never read the
        # buffer the previous op just streamed (no reuse through the 256 MB MALL).
        def make_step(i):
            seq = [calls[(len(ops4) * i + j) % nbuf][j] for j in range(len(ops4))]

            def f():
                for c in seq:
                    c()
            return f

        step_fns = [make_step(i) for i in range(nbuf)]
        ms_step = time_calls(torch, step_fns, steps, warmup)
        value = step_bytes / (ms_step * 1e-3) / 1e9

        breakdown = {}
        for j, op in enumerate(ops4):
            fns = [calls[i][j] for i in range(nbuf)]
            ms = time_calls(torch, fns, steps, warmup)
            gbs = op_bytes[j] / (ms * 1e-3) / 1e9
            breakdown[op] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
                             "alg_bytes": op_bytes[j], "kernel": DOMINANT_KERNEL[op]}
        dom_name, dom = max(breakdown.items(), key=lambda kv: kv[1]["ms"])
        dom_j = ops4.index(dom_name)
        dom_ms = dom["ms"]  # average launch duration over the timed loop of that op alone
        dom_gbs = op_bytes[dom_j] / (dom_ms * 1e-3) / 1e9

        traffic = None
        if os.path.exists(args.traffic_file):
            try:
                tf = json.load(open(args.traffic_file))
                traffic = tf.get("C4_" + dom_name, {}).get("hbm_bytes_per_launch")
            except Exception:
                traffic = None
        result.update({"value": round(value, 1), "ms_per_step": round(ms_step, 5)})
        result["config"]["frac_of_peak"] = round(value / HBM_PEAK_GBS, 4)
        result["roofline"] = {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                              "op": dom_name, "kernel": DOMINANT_KERNEL.get(dom_name, "?"),
                              "avg_launch_ms": round(dom_ms, 5), "alg_bytes_per_launch": op_bytes[dom_j],
                              "timing": "HIP events on the launch stream, average over the op's own timed loop"}
        result["breakdown"] = breakdown

    keep = {"C4": bufs[0]}
    result["configs"] = run_sections(torch, capi, only, stream, steps, warmup, keep)
    if args.calibrate_copy:
        xc = gen(torch, (64 << 20,), "normal", 6000, dev)
        for _ in range(3):
            capi.copy_strided(xc)
        torch.cuda.synchronize()

    # ---------------- CPU baseline and accuracy (rank 0, N = 1) -------------------
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(bufs[0], ops4, op_bytes)
        result["cpu_baseline"]["configs"] = cpu_extras(keep.get("C2"), keep.get("C3"), keep.get("C5"))
    else:
        result["cpu_baseline"] = None
    if not args.no_accuracy:
        result["accuracy"] = accuracy(torch, capi, keep)
    if args.vs_torch:
        del keep, bufs, calls, step_fns
        result["torch_rocm"] = torch_rocm_times(torch, steps, warmup)
    print(json.dumps(result), flush=True)


def torch_rocm_times(torch, steps, warmup):
    """PyTorch-ROCm's own kernels on the same shapes and rotating inputs, timed
    the same way (HIP events; `GB/s` = the same algorithmic bytes as ours)."""
    dev = torch.device("cuda:0")
    bufs = [gen(torch, (64, 1024, 1024), "normal", 1000 + i, dev) for i in range(3)]
    out = {}

    def t(name, fns, by):
        out[name] = rate(time_calls(torch, fns, max(steps, 10), warmup), by)

    n2 = 64 * 1024 * 1024 * 4
    t("C2_mean_dim1", [lambda b=b: b.mean(1) for b in bufs], n2 + 64 * 1024 * 4)
    t("C2_amax_dim0", [lambda b=b: b.amax(0) for b in bufs], n2 + 1024 * 1024 * 4)
    t("C2_argmax_dim0", [lambda b=b: b.argmax(0) for b in bufs], n2 + 1024 * 1024 * 8)
    t("C2_var_dim-1", [lambda b=b: b.var(-1) for b in bufs], n2 + 64 * 1024 * 4)
    t("C2_std_dim-1", [lambda b=b: b.std(-1) for b in bufs], n2 + 64 * 1024 * 4)
    t("C2_clone", [lambda b=b: b.clone() for b in bufs], 2 * n2)
    t("C2_permute_1_2_0", [lambda b=b: b.permute(1, 2, 0).contiguous() for b in bufs], 2 * n2)
    t("C2_to_float64", [lambda b=b: b.to(torch.float64) for b in bufs], 3 * n2)
    b1 = [gen(torch, (4096, 4096), "normal", 2000 + i, dev) for i in range(12)]
    t("C1_sum_dim-1", [lambda b=b: b.sum(-1) for b in b1], 4096 * 4096 * 4 + 4096 * 4)
    del b1
    b3 = [gen(torch, (1024, 32768), "uniform", 3000 + i, dev) for i in range(6)]
    t("C3_topk64", [lambda b=b: torch.topk(b, 64, dim=1) for b in b3], 1024 * 32768 * 4 + 1024 * 64 * 12)
    t("C3_softmax", [lambda b=b: torch.softmax(b, -1) for b in b3[:4]], 2 * 1024 * 32768 * 4)
    del b3
    del bufs
    x4 = [gen(torch, (1 << 28,), "normal", 4000 + i, dev) * 2.0 + 0.5 for i in range(3)]
    for op in ("sum", "amax", "argmax", "var"):
        t(f"C4_{op}", [lambda b=b, op=op: getattr(b, op)() for b in x4], (1 << 28) * 4 + 8)
    del x4
    b5 = [gen(torch, (256, 151936), "normal", 5000 + i, dev) * 3.0 for i in range(5)]
    n5 = 256 * 151936 * 4
    t("C5_topk50", [lambda b=b: torch.topk(b, 50, dim=1) for b in b5], n5 + 256 * 50 * 12)
    t("C5_argmax_dim-1", [lambda b=b: b.argmax(-1) for b in b5], n5 + 256 * 8)
    t("C5_softmax", [lambda b=b: torch.softmax(b, -1) for b in b5[:3]], 2 * n5)
    t("C5_log_softmax", [lambda b=b: torch.log_softmax(b, -1) for b in b5[:3]], 2 * n5)
    del b5
    b6 = [gen(torch, (4096, 2048), "uniform", 7000 + i, dev) for i in range(3)]
    t("topk1000_4096x2048", [lambda b=b: torch.topk(b, 1000, dim=1) for b in b6], 4096 * 2048 * 4 + 4096 * 1000 * 12)
    del b6
    return out


def timed(torch, calls, steps, warmup, by, **extra):
    ms = time_calls(torch, calls, steps, warmup)
    return dict(rate(ms, by), **extra)


def run_sections(torch, capi, only, stream, steps, warmup, keep):
    """The other BASELINE configs and the widened rows, each timed the same way
    (HIP events, inputs rotated so each launch reads HBM)."""
    dev = keep["C4"].device
    extras = {}
    nbuf = 3
    need_c2 = only & {"C2", "copy", "reduce_backward", "softmax_cols"}
    bufs = [gen(torch, (64, 1024, 1024), "normal", 1000 + i, dev) for i in range(nbuf)] if need_c2 else []
    if bufs:
        keep["C2"] = bufs[0]
    if "C2" in only:
        # C2: strided reductions of [64,1024,1024] N(0,1): mean dim=1, amax+argmax dim=0, var+std dim=-1
        ops2 = [("mean", [1]), ("amax", [0]), ("argmax", [0]), ("var", [-1]), ("std", [-1])]
        c2 = [[reduce_call(torch, capi, b, op, dims, stream) for (op, dims) in ops2] for b in bufs]
        ob = [64 * 1024 * 1024 * 4 + c.out_bytes for c in c2[0]]

        def make_step(i):
            seq = [c2[(len(ops2) * i + j) % nbuf][j] for j in range(len(ops2))]

            def f():
                for c in seq:
                    c()
            return f

        ms = time_calls(torch, [make_step(i) for i in range(nbuf)], steps, warmup)
        e2 = {"step": rate(ms, sum(ob))}
        for j, (op, dims) in enumerate(ops2):
            name = f"{op}_dim{dims[0]}"
            e2[name] = timed(torch, [c2[i][j] for i in range(nbuf)], steps, warmup, ob[j], kernel=C2_KERNEL[name])
        extras["C2_strided_64x1024x1024"] = e2
        del c2

    if "C1" in only:
        # C1: sum dim=-1 of [4096,4096] (12 rotating 64 MiB buffers)
        b1 = [gen(torch, (4096, 4096), "normal", 2000 + i, dev) for i in range(12)]
        c1 = [reduce_call(torch, capi, b, "sum", [-1], stream) for b in b1]
        by = 4096 * 4096 * 4 + c1[0].out_bytes
        extras["C1_sum_dim-1_4096x4096"] = timed(torch, c1, max(steps, 24) * 4, warmup, by,
                                                 kernel="k_rows_reg<SumOp,2,8,512>")
        keep["C1"] = b1[0]
        del b1, c1
    if "C3" in only or "softmax" in only:
        b3 = [gen(torch, (1024, 32768), "uniform", 3000 + i, dev) for i in range(6)]
        keep["C3"] = b3[0]
        if "C3" in only:
            # C3: topk k=64 of [1024,32768] U(-1,1)
            c3 = [topk_call(torch, capi, b, 64, stream) for b in b3]
            by = 1024 * 32768 * 4 + c3[0].out_bytes
            r = timed(torch, c3, max(steps, 12), warmup, by)
            r["rows_per_s"] = round(1024 / (r["ms"] * 1e-3), 1)
            extras["C3_topk64_1024x32768"] = r
            del c3
        if "softmax" in only:
            # softmax / log_softmax along the rows of the same tensors (register-resident rows)
            esm3 = {}
            for name, mode in (("softmax", capi.SOFTMAX_FWD), ("log_softmax", capi.LOG_SOFTMAX_FWD)):
                cs = [softmax_call(torch, capi, b, -1, mode, stream) for b in b3[:4]]
                esm3[name] = timed(torch, cs, max(steps, 12), warmup, cs[0].bytes)
                del cs
            extras["softmax_C3_1024x32768"] = esm3
        del b3
    if "C4f64" in only:
        # the same 1 GiB as float64 (2^27 elements): reductions computed in double
        x4d = gen(torch, (1 << 27,), "normal", 4001, dev).double() * 2.0 + 0.5
        c4d = {}
        for op in ("sum", "amax", "argmax", "var"):
            c = reduce_call(torch, capi, x4d, op, None, stream)
            c4d[op] = timed(torch, [c], max(steps // 2, 5), 2, (1 << 27) * 8 + c.out_bytes)
        extras["C4_full_f64_2^27"] = c4d
        del x4d
    if "C5" in only or "softmax" in only:
        # C5: [256,151936] N(0,3) + 8 boosted positions per row
        b5 = []
        for i in range(5):
            x = gen(torch, (256, 151936), "normal", 5000 + i, dev) * 3.0
            g = torch.Generator(device="cpu")
            g.manual_seed(5100 + i)
            pos = torch.stack([torch.randperm(151936, generator=g)[:8] for _ in range(256)]).to(dev)
            x.scatter_add_(1, pos, torch.full((256, 8), 15.0, device=dev))
            b5.append(x)
        keep["C5"] = b5[0]
        if "C5" in only:
            c5 = [topk_call(torch, capi, b, 50, stream) for b in b5]
            by = 256 * 151936 * 4 + c5[0].out_bytes
            e5 = {"topk50": timed(torch, c5, max(steps, 10), warmup, by)}
            e5["topk50"]["rows_per_s"] = round(256 / (e5["topk50"]["ms"] * 1e-3), 1)
            c5a = [reduce_call(torch, capi, b, "argmax", [-1], stream) for b in b5]
            e5["argmax_dim-1"] = timed(torch, c5a, max(steps, 10), warmup, 256 * 151936 * 4 + c5a[0].out_bytes)
            # top-k (k=50) -> top-p (0.9) sampling of one token per row, T = 0.7
            uu = torch.rand((256,), device=dev)
            cs = [sample_call(torch, capi, b, 50, 0.7, 0.9, uu, stream) for b in b5]
            e5["sample_topk50_topp0.9"] = timed(torch, cs, max(steps, 10), warmup, cs[0].bytes)
            e5["sample_topk50_topp0.9"]["rows_per_s"] = round(256 / (e5["sample_topk50_topp0.9"]["ms"] * 1e-3), 1)
            extras["C5_logits_256x151936"] = e5
            del c5, c5a, cs
        if "softmax" in only:
            # softmax / log_softmax forward (read + write), their gradients (read g and y, write the
            # gradient), and nll_loss backward (write [256, 151936])
            esm = {}
            for name, mode in (("softmax", capi.SOFTMAX_FWD), ("log_softmax", capi.LOG_SOFTMAX_FWD)):
                cs = [softmax_call(torch, capi, b, -1, mode, stream) for b in b5[:3]]
                esm[name] = timed(torch, cs, max(steps, 10), warmup, cs[0].bytes)
                del cs
            for name, mode in (("softmax_backward", capi.SOFTMAX_BWD),
                               ("log_softmax_backward", capi.LOG_SOFTMAX_BWD)):
                cs = [softmax_call(torch, capi, b5[i], -1, mode, stream, y=b5[i + 1]) for i in (0, 2)]
                esm[name] = timed(torch, cs, max(steps, 10), warmup, cs[0].bytes)
                del cs
            tgt = torch.randint(0, 151936, (256,), device=dev, dtype=torch.int64)
            one = torch.ones((), device=dev)
            tw = torch.full((1,), 256.0, device=dev)
            cs = [nll_bwd_call(torch, capi, 256, 151936, tgt, one, tw, stream) for _ in range(3)]
            esm["nll_loss_backward"] = timed(torch, cs, max(steps, 10), warmup, cs[0].bytes)
            del cs
            extras["softmax_C5_logits_256x151936"] = esm
        del b5
    if "copy" in only:
        # copy_ (strided / casting) on the C2 geometry: read + write bytes
        ecp = {}
        cases = {"permute_1_2_0": (lambda b: b.permute(1, 2, 0), torch.float32),
                 "transpose_1_2": (lambda b: b.transpose(1, 2), torch.float32),
                 "clone_dense": (lambda b: b, torch.float32),
                 "cast_f32_to_f64": (lambda b: b, torch.float64)}
        for name, (view, odt) in cases.items():
            outs = [torch.empty(view(bufs[0]).shape, dtype=odt, device=dev) for _ in range(2)]
            cc = [copy_call(torch, capi, outs[i % 2], view(bufs[i % nbuf]), stream) for i in range(6)]
            ecp[name] = timed(torch, cc, max(steps, 12), warmup, cc[0].bytes,
                              kernel=copy_kernel_name(capi.copy_plan(outs[0], view(bufs[0]))))
            del outs, cc
        extras["copy_C2_64x1024x1024"] = ecp
    if "reduce_backward" in only:
        # gradients of the C2 reductions (var / std over dim=-1, mean over dim=1) and of a full sum
        erb = {}
        for op, dims in (("var", [-1]), ("std", [-1]), ("mean", [1]), ("sum", None)):
            nd = 3
            rd = list(range(nd)) if dims is None else [d % nd for d in dims]
            kept = [bufs[0].shape[i] for i in range(nd) if i not in rd]
            g = torch.randn(kept, device=dev)
            res = torch.rand(kept, device=dev) + 0.5 if op == "std" else None
            cs = [reduce_bwd_call(torch, capi, bufs[i], op, dims, stream, g, res) for i in range(nbuf)]
            erb[f"{op}_backward_dim{'' if dims is None else dims[0]}"] = timed(torch, cs, max(steps, 9), warmup,
                                                                                 cs[0].bytes)
            del cs
        extras["reduce_backward_C2_64x1024x1024"] = erb
    if "softmax_cols" in only:
        # softmax over the middle (strided) dim of the C2 geometry
        cs = [softmax_call(torch, capi, bufs[i], 1, capi.SOFTMAX_FWD, stream) for i in range(2)]
        extras["softmax_C2_dim1_64x1024x1024"] = timed(torch, cs, max(steps, 8), warmup, cs[0].bytes)
        del cs
    if "topk_short" in only:
        # many short rows (lane groups per row), a large k (rows held in registers) and k = 256 over C5-sized
        # vocabulary rows (the wave kernel's 512-entry lists), beside the BASELINE top-k configs; int32 rows
        # (full-range values: the float filter kernels on integer keys) and int8 rows (register radix select)
        ets = {}
        for (rows, cols, k, dt) in ((65536, 256, 8, "f32"), (16384, 1024, 32, "f32"), (4096, 2048, 1000, "f32"),
                                    (256, 151936, 256, "f32"), (16384, 1024, 32, "i32"), (1024, 32768, 64, "i32"),
                                    (16384, 1024, 32, "i8"), (256, 151936, 50, "i8"), (256, 151936, 50, "f64")):
            esz = {"f32": 4, "i32": 4, "i8": 1, "f64": 8}[dt]
            nb = max(3, (768 << 20) // (rows * cols * esz))
            bs = [gen(torch, (rows, cols), "uniform", 7000 + i, dev) for i in range(nb)]
            if dt == "i32":
                bs = [(b * 2.0 ** 31).clamp(-2.0 ** 31, 2.0 ** 31 - 1).to(torch.int32) for b in bs]
            elif dt == "i8":
                bs = [(b * 127.0).round().to(torch.int8) for b in bs]
            elif dt == "f64":
                bs = [b.double() for b in bs]
            cs = [topk_call(torch, capi, b, k, stream) for b in bs]
            r = timed(torch, cs, max(steps, 12), warmup, rows * cols * esz + cs[0].out_bytes)
            r["rows_per_s"] = round(rows / (r["ms"] * 1e-3), 1)
            ets[f"topk{k}_{rows}x{cols}" + ("" if dt == "f32" else "_" + {"i32": "int32", "i8": "int8", "f64": "float64"}[dt])] = r
            del bs, cs
        extras["topk_short_rows"] = ets
    return extras


def _err_stats(got, ref, x_abs_sum=None):
    """Max and median relative error of `got` against the fp64 `ref`, and the
    normwise error max |got - ref| / sum |x| over each output's inputs."""
    import numpy as np
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    out = {"max_rel": float(f"{rel.max():.3e}"), "median_rel": float(f"{np.median(rel):.3e}")}
    if x_abs_sum is not None:
        nw = np.abs(got - ref) / np.maximum(np.asarray(x_abs_sum, np.float64).reshape(-1), 1e-30)
        out["normwise"] = float(f"{nw.max():.3e}")
    return out


def accuracy(torch, capi, keep):
    """Error of this backend's GPU result and of TensorPlay's CPU path (the C
    restatement in oracle/, same input) against an fp64 host reference, per op
    and config (north_star: <= 1e-5 relative for fp32 sum/mean/var/std,
    reported beside the CPU path's own error)."""
    import numpy as np
    from oracle import oracle as O

    def gpu(t, op, dims):
        r = capi.reduce(t, op, dims)
        torch.cuda.synchronize()
        return r.cpu().numpy()

    acc = {"reference": "numpy float64 on the same fp32 input; cpu_path = oracle/tp_cpu_reduce.c "
                        "(TensorPlay's CPU reduction order and accumulation types)",
           "bound": "gpu max_rel <= 1e-5"}
    if "C1" in keep:
        x = keep["C1"].cpu().numpy()
        x64 = x.astype(np.float64)
        ref, asum = x64.sum(1), np.abs(x64).sum(1)
        acc["C1_sum_dim-1"] = {"gpu": _err_stats(gpu(keep["C1"], "sum", [-1]), ref, asum),
                               "cpu_path": _err_stats(O.sum(x, [-1]), ref, asum)}
    if "C2" in keep:
        x = keep["C2"].cpu().numpy()
        x64 = x.astype(np.float64)
        ref, asum = x64.mean(1), np.abs(x64).mean(1)
        c2 = {"mean_dim1": {"gpu": _err_stats(gpu(keep["C2"], "mean", [1]), ref, asum),
                            "cpu_path": _err_stats(O.mean(x, [1]), ref, asum)}}
        v = x64.var(2, ddof=1)
        c2["var_dim-1"] = {"gpu": _err_stats(gpu(keep["C2"], "var", [-1]), v), "cpu_path": _err_stats(O.var(x, [-1]), v)}
        c2["std_dim-1"] = {"gpu": _err_stats(gpu(keep["C2"], "std", [-1]), np.sqrt(v)),
                           "cpu_path": _err_stats(O.std(x, [-1]), np.sqrt(v))}
        acc["C2"] = c2
        del x, x64
    if "C4" in keep:
        x = keep["C4"].cpu().numpy()
        x64 = x.astype(np.float64)
        s, asum = x64.sum(), np.abs(x64).sum()
        m = s / x.size
        v = x64.var(ddof=1)
        del x64
        c4 = {"sum": {"gpu": _err_stats(gpu(keep["C4"], "sum", None), s, asum),
                      "cpu_path": _err_stats(O.sum(x), s, asum)},
              "mean": {"gpu": _err_stats(gpu(keep["C4"], "mean", None), m, asum / x.size),
                       "cpu_path": _err_stats(O.mean(x), m, asum / x.size)},
              "var": {"gpu": _err_stats(gpu(keep["C4"], "var", None), v), "cpu_path": _err_stats(O.var(x), v)},
              "std": {"gpu": _err_stats(gpu(keep["C4"], "std", None), np.sqrt(v)),
                      "cpu_path": _err_stats(O.std(x), np.sqrt(v))}}
        acc["C4"] = c4
    return acc


def cpu_baseline(x_dev, ops4, op_bytes, budget_s=12.0):
    """Time the C restatement of TensorPlay's CPU reduction path (single-threaded,
    as ReductionKernels.cpp is) on the headline step: the same six full
    reductions of one 1 GiB buffer copied to host memory, repeated until
    ~budget_s (at least one whole step)."""
    from oracle import oracle as O

    x = x_dev.cpu().numpy()
    fns = {"sum": lambda: O.sum(x), "mean": lambda: O.mean(x), "amax": lambda: O.amax(x),
           "argmax": lambda: O.argmax(x, None), "var": lambda: O.var(x), "std": lambda: O.std(x)}
    per = {op: 0.0 for op in ops4}
    reps = 0
    t0 = time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < budget_s:
        for op in ops4:
            t = time.perf_counter()
            fns[op]()
            per[op] += time.perf_counter() - t
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    total = float(sum(op_bytes))
    return {"value": round(total / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{reps} full headline steps (sum, mean, amax, argmax, var, std of one 2^28-element "
                      "buffer) through oracle/tp_cpu_reduce.c, 1 thread",
            "seconds_per_step": round(dt, 4),
            "per_op_s": {k: round(v / reps, 4) for k, v in per.items()}, "host_cpus": os.cpu_count()}


def cpu_extras(c2_dev, c3_dev, c5_dev):
    """CPU figures for the other configs on bounded samples (1 thread unless noted)."""
    import numpy as np
    from oracle import oracle as O

    out = {}
    if c2_dev is not None:
        x2 = c2_dev.cpu().numpy()
        t = time.perf_counter()
        O.mean(x2, [1]), O.amax(x2, [0]), O.argmax(x2, 0), O.var(x2, [-1]), O.std(x2, [-1])
        dt = time.perf_counter() - t
        out["C2_strided_step"] = {"GB/s": round(5 * x2.nbytes / dt / 1e9, 3), "cores": 1,
                                  "sample": "one step: mean dim1, amax+argmax dim0, var+std dim-1 of one buffer"}
    x1 = np.random.default_rng(1).standard_normal((4096, 4096), dtype=np.float32)
    t = time.perf_counter()
    O.sum(x1, [-1])
    dt = time.perf_counter() - t
    out["C1_sum_dim-1_4096x4096"] = {"GB/s": round(x1.nbytes / dt / 1e9, 3), "sample": "full config", "cores": 1}
    if c3_dev is None or c5_dev is None:
        return out
    x3 = c3_dev[:256].cpu().numpy()
    t = time.perf_counter()
    O.topk(x3, 64)
    dt = time.perf_counter() - t
    out["C3_topk64_1024x32768"] = {"GB/s": round(x3.nbytes / dt / 1e9, 3), "rows_per_s": round(256 / dt, 1),
                                   "sample": "256 of 1024 rows, heap selection + sort (no TensorPlay topk exists)",
                                   "cores": 1}
    nt = min(16, os.cpu_count() or 1)
    t = time.perf_counter()
    O.topk(x3, 64, threads=nt)
    dt = time.perf_counter() - t
    out["C3_topk64_1024x32768"]["all_cores"] = {"GB/s": round(x3.nbytes / dt / 1e9, 3), "cores": nt}
    x5 = c5_dev[:64].cpu().numpy()
    t = time.perf_counter()
    O.topk(x5, 50)
    dt = time.perf_counter() - t
    out["C5_topk50_256x151936"] = {"GB/s": round(x5.nbytes / dt / 1e9, 3), "rows_per_s": round(64 / dt, 1),
                                   "sample": "64 of 256 rows", "cores": 1}
    t = time.perf_counter()
    O.argmax(x5, -1)
    dt = time.perf_counter() - t
    out["C5_argmax_dim-1"] = {"GB/s": round(x5.nbytes / dt / 1e9, 3), "sample": "64 of 256 rows", "cores": 1}
    return out


if __name__ == "__main__":
    main()
