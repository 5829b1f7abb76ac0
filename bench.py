"""CSR SpMV benchmark on one MI355X: y = alpha*op(A)*x + beta*y through aclsparseSpMV.

A step is one aclsparseSpMV over the whole matrix (Preprocess runs once before
timing and is reported separately).  Before every timed step a 512 MiB buffer
is read so that A, x and y come from HBM, not from L2 / MALL; the SpMV
itself is timed with HIP events recorded on the stream it runs on.  c1
(1.4 MB, launch-bound) is also timed as 1000 back-to-back SpMVs replayed
from one HIP graph.

The headline workload is the largest configuration of BASELINE.json
(configs[3], c4): 16,777,216 x 16,777,216 with 32 uniform columns per row
(536,870,912 non-zeros), fp16 values and x, fp32 compute, fp16 output, int64
row offsets.  The other configurations (c1, c2, c3, c4 in bf16, c5, and the
headline-matrix variants of c2) are measured in the same run (``configs``
field) unless ``--only-headline`` is given.

Prints ONE JSON line.
"""
import argparse
import json
import os
import platform
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "ops-sparse_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
HEADLINE = "c4h"  # BASELINE.json configs[3] in fp16: the largest configuration
METRIC = "CSR SpMV GFLOP/s + effective HBM GB/s (% of MI355X peak) on one GPU"
FLUSH_BYTES = 512 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--configs", default="c1,c2,c3,c4h,c4b,c5")
    ap.add_argument("--profile", default=None,
                    help="profiling mode: build only this config, run --steps SpMVs and a 1 GiB copy "
                         "(the calibration kernel for FETCH_SIZE/WRITE_SIZE), print nothing else")
    return ap.parse_args()


def profile_mode(name, steps):
    """Minimal launch sequence for rocprofv3: Preprocess once, ``steps`` SpMVs, one 1 GiB device copy."""
    from ops_sparse.spmv import CsrSpMV
    from ops_sparse._lib import Operation
    from ops_sparse.workloads import algorithmic_bytes

    dev = torch.device("cuda:0")
    if name.startswith("spmm"):
        from ops_sparse.spmm import SpMMOp
        from ops_sparse import workloads as wl

        case = dict(spmm_cases(dev, wl.config("c2", dev)))[name]
        op = SpMMOp(case["m"], case["k"], case["rp"], case["col"], case["val"], case["b"], case["c"])
        for _ in range(steps):
            op.run(case["b"], case["c"], case["alpha"], case["beta"])
        torch.cuda.synchronize()
        return
    if name.startswith("c2_spmvop_"):
        from ops_sparse.spmv import SpMVOp
        from ops_sparse._lib import SpMVOpAlg
        from ops_sparse import workloads as wl

        w = wl.config("c2", dev)
        z = torch.empty_like(w.y0)
        op = SpMVOp(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, w.y0, z,
                    alg=getattr(SpMVOpAlg, name[len("c2_spmvop_"):].upper()))
        for _ in range(steps):
            op.run(w.alpha, w.beta)
        torch.cuda.synchronize()
        op.close()
        return
    w = make(name, dev)
    y = w.y0.to(w.out_dtype).clone()
    op = {"N": Operation.NON_TRANSPOSE, "T": Operation.TRANSPOSE, "H": Operation.CONJUGATE_TRANSPOSE}[w.trans]
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=op)
    plan.preprocess()
    torch.cuda.synchronize()  # as in a bench run: Preprocess's path choice is on the host before the SpMVs
    flush_buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
    sink = torch.empty((), dtype=torch.float32, device=dev)
    for _ in range(steps):
        torch.sum(flush_buf, dim=0, out=sink)  # same L2/MALL state as a bench step
        plan.run()
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)  # 1 GiB read + 1 GiB write: scales the per-dispatch counters
    torch.cuda.synchronize()
    print(json.dumps({"profile": name, "workload": w.name, "algorithmic_bytes": algorithmic_bytes(w),
                      "copy_bytes_each_way": src.numel() * 4, "steps": steps}))


def dtype_variants(w):
    """The headline matrix through the other paths of the dtype/op matrix (same sparsity)."""
    from ops_sparse.workloads import Workload

    g = torch.Generator(device=w.values.device)
    g.manual_seed(99)
    n = w.nnz

    def i8(k):
        return torch.randint(-128, 128, (k,), generator=g, device=w.values.device, dtype=torch.int8)

    def c64(v):
        return torch.complex(v, 0.5 * v.flip(0))

    out = {
        "c2_T": Workload(w.name + "_T", w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, w.y0, 1.5, 0.5,
                         trans="T"),
        "c2_f16": Workload(w.name + "_f16", w.rows, w.cols, w.row_ptr, w.col_ind, w.values.half(), w.x.half(),
                           w.y0.half(), 1.5, 0.5, out_dtype=torch.float16),
        "c2_i8": Workload(w.name + "_i8", w.rows, w.cols, w.row_ptr, w.col_ind, i8(n), i8(w.cols),
                          torch.randint(-1000, 1000, (w.rows,), generator=g, device=w.values.device,
                                        dtype=torch.int32), 2, 1, out_dtype=torch.int32),
        "c2_c64": Workload(w.name + "_c64", w.rows, w.cols, w.row_ptr, w.col_ind, c64(w.values), c64(w.x),
                           c64(w.y0), 1.5, 0.5, out_dtype=torch.complex64),
    }
    out["c2_c64_H"] = Workload(w.name + "_c64_H", w.rows, w.cols, w.row_ptr, w.col_ind, out["c2_c64"].values,
                               out["c2_c64"].x, out["c2_c64"].y0, 1.5, 0.5, trans="H", out_dtype=torch.complex64)
    return out


def make(name, dev):
    from ops_sparse import workloads as wl

    if name == "c4h":
        return wl.uniform_rows_lowp(device=dev, dtype=torch.float16)
    if name == "c4b":
        return wl.uniform_rows_lowp(device=dev, dtype=torch.bfloat16)
    if name.startswith("c2_") and not name.startswith("c2_spmvop"):
        return dtype_variants(wl.config("c2", dev))[name]
    return wl.config(name, dev)


def _timed(stream, fn, reps):
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def measure(w, steps, warmup, flush_buf, alg=None):
    """SpMV time per step (ms) with L2/MALL flushed before every SpMV.

    A step is a read of a 512 MiB buffer (evicting the L2 and the 256 MB
    MALL) followed by one SpMV, so the SpMV starts with its inputs in HBM
    only.  ``median_ms`` is the median over ``steps`` of an event pair around
    each SpMV launch on the launch stream: it agrees with the kernel
    duration rocprofv3 reports for the same launches (it includes the
    dispatch latency of one launch, a few microseconds).  For reference only:
    ``dirty_flush_ms`` (the same after a read-modify-write flush, whose dirty
    lines the SpMV then has to write back), ``paired_ms`` (back-to-back
    flush+SpMV steps minus flushes alone) and ``warm_ms`` (back-to-back
    SpMVs, L2/MALL warm).
    """
    from ops_sparse.spmv import CsrSpMV
    from ops_sparse._lib import Operation

    from ops_sparse._lib import SpMVAlg

    op = {"N": Operation.NON_TRANSPOSE, "T": Operation.TRANSPOSE, "H": Operation.CONJUGATE_TRANSPOSE}[w.trans]
    y = w.y0.to(w.out_dtype).clone()
    plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=op,
                   alg=SpMVAlg.DEFAULT if alg is None else alg)
    stream = torch.cuda.current_stream()
    # Preprocess: the median of three calls after a first one (the first
    # Preprocess of a process also pays for loading code objects)
    plan.preprocess()
    torch.cuda.synchronize()
    pre = []
    for _ in range(3):
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p0.record(stream)
        plan.preprocess()
        p1.record(stream)
        torch.cuda.synchronize()
        pre.append(p0.elapsed_time(p1))
    pre_ms = statistics.median(pre)
    # the path Preprocess chose: the path flag in the workspace header
    path = "row kernels" if w.trans == "N" else "transpose"
    if w.trans == "N" and plan.workspace is not None and plan.workspace.numel() >= 192:
        head = np.frombuffer(plan.workspace[:192].cpu().numpy().tobytes(), dtype=np.uint64)
        path = {1: "staged gather", 3: NARROW_PATH, 5: NARROW_PATH}.get(int(head[16] & 0xFFFFFFFF), path)

    sink = torch.empty((), dtype=torch.float32, device=flush_buf.device)

    def flush():
        # read-only: evicts L2/MALL without leaving dirty lines whose
        # write-back the next kernel would pay for
        torch.sum(flush_buf, dim=0, out=sink)

    def step():
        flush()
        plan.run()

    for _ in range(warmup):
        step()
    rounds = 5
    per_round = max(1, steps // rounds)
    diffs = []
    t0 = time.perf_counter()
    for _ in range(rounds):
        both = _timed(stream, step, per_round)
        alone = _timed(stream, flush, per_round)
        diffs.append(both - alone)
    wall = (time.perf_counter() - t0) * 1e3 / (rounds * per_round)
    # one event pair per launch (includes the launch latency)
    def per_launch(pre):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in evs:
            pre()
            a.record(stream)
            plan.run()
            b.record(stream)
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(b) for a, b in evs)
        return statistics.median(ts), ts[min(len(ts) - 1, (9 * len(ts)) // 10)]

    ev, ev_p90 = per_launch(flush)
    # reference: after a 512 MiB read-modify-write flush, the SpMV also pays
    # for writing back the flush's dirty L2/MALL lines
    ev_dirty, _ = per_launch(lambda: flush_buf.add_(1))
    # back-to-back launches without a flush (L2/MALL warm), for reference only
    warm = _timed(stream, plan.run, steps)
    return dict(median_ms=ev, p90_ms=ev_p90, dirty_flush_ms=ev_dirty, paired_ms=statistics.median(diffs), paired_min_ms=min(diffs),
                paired_max_ms=max(diffs), wall_ms_per_step=wall, warm_ms=warm, preprocess_ms=pre_ms,
                workspace_bytes=plan.buffer_size, path=path)


def graph_ms(w, launches=1000, replays=5):
    """Per-SpMV time (ms) of ``launches`` back-to-back SpMVs captured in one HIP graph.

    For launch-bound sizes: the graph removes the host dispatch cost, so the
    figure is the GPU's own time per SpMV (L2-resident inputs).  The plan is
    built and preprocessed on the capture stream (a stream change would
    invalidate it); the SpMV enqueues only kernels, no memsets or copies.
    """
    from ops_sparse.spmv import CsrSpMV
    from ops_sparse._lib import Operation

    op = Operation.NON_TRANSPOSE if w.trans == "N" else Operation.TRANSPOSE
    y = w.y0.to(w.out_dtype).clone()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        plan = CsrSpMV(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, y, w.alpha, w.beta, op=op)
        plan.preprocess()
        plan.run()
    torch.cuda.synchronize()
    ref = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(launches):
            plan.run()
    # a replay must recompute y from scratch (beta = 0) or accumulate into it
    y.zero_()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    if w.beta == 0 and not torch.equal(y, ref):
        raise RuntimeError("the captured graph does not reproduce the SpMV")
    ts = []
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):  # replay() launches on the current stream
            a.record(s)
            g.replay()
            b.record(s)
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / launches)
        if w.beta == 0 and not torch.equal(y, ref):
            raise RuntimeError("graph replay changed the SpMV result")
    return statistics.median(ts)


def measure_spmvop(w, alg, steps, warmup, flush_buf):
    """aclsparseSpMVOp (Z = alpha*A*X + beta*Y, compensated fp32 dot) on the same matrix:
    median per-launch time (ms) after the same read-only flush, and the set-up time
    (bufferSize, the buffer from torch's caching allocator, createDescr with its table
    kernels, createPlan), by events on the stream: a first set-up in the process
    (code objects loaded, the buffer newly allocated) and a second one after it."""
    from ops_sparse.spmv import SpMVOp

    z = torch.empty_like(w.y0)
    stream = torch.cuda.current_stream()
    setups = []
    for _ in range(2):
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p0.record(stream)
        op = SpMVOp(w.rows, w.cols, w.row_ptr, w.col_ind, w.values, w.x, w.y0, z, alg=alg)
        p1.record(stream)
        torch.cuda.synchronize()
        setups.append(p0.elapsed_time(p1))
        if len(setups) == 1:
            op.close()
            del op
    sink = torch.empty((), dtype=torch.float32, device=flush_buf.device)
    for _ in range(warmup):
        torch.sum(flush_buf, dim=0, out=sink)
        op.run(w.alpha, w.beta)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        torch.sum(flush_buf, dim=0, out=sink)
        a.record(stream)
        op.run(w.alpha, w.beta)
        b.record(stream)
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in evs)
    op.close()
    return statistics.median(ts), setups


def spmm_cases(dev, headline_w):
    """SpMMOp workloads: the largest shape of the reference's own SpMMOp perf table
    (test/spmm_op/arch35/spmm_op_perf.cpp:740-790: M=2048, K=128, N=2048, 50% density,
    alpha=1, beta=0, fp32 and fp16, L2-resident, timed warm as there) and the headline
    Laplacian times a 16-column dense block (HBM-sized, flushed like the SpMV configs)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np

    out = []
    m, k, n = 2048, 128, 2048
    thr = 50
    mask = ((np.arange(m) % 100)[:, None] * 7 + (np.arange(k) % 100)[None, :] * 13) % 100 < thr
    rows, cols = np.nonzero(mask)
    rp = np.zeros(m + 1, np.int32)
    rp[1:] = np.cumsum(mask.sum(axis=1))
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    for dt, tag in ((torch.float32, "fp32"), (torch.float16, "fp16")):
        vals = (torch.rand(rows.size, generator=g, device=dev) * 2 - 1).to(dt)
        b = (torch.rand(k, n, generator=g, device=dev) * 2 - 1).to(dt)
        c = torch.zeros(m, n, dtype=dt, device=dev)
        out.append((f"spmm_ref_2048x128x2048_{tag}_sp50",
                    dict(m=m, k=k, n=n, rp=torch.from_numpy(rp).to(dev), col=torch.from_numpy(cols.astype(np.int32)).to(dev),
                         val=vals, b=b, c=c, alpha=1.0, beta=0.0, flush=False)))
    w = headline_w
    n2 = 16
    b = torch.rand(w.cols, n2, generator=g, device=dev) * 2 - 1
    c = torch.rand(w.rows, n2, generator=g, device=dev) * 2 - 1
    out.append((f"spmm_c2_laplacian_x{n2}_fp32", dict(m=w.rows, k=w.cols, n=n2, rp=w.row_ptr, col=w.col_ind,
                                                      val=w.values, b=b, c=c, alpha=1.5, beta=0.5, flush=True)))
    return out


def measure_spmm(case, steps, warmup, flush_buf):
    """Median per-launch time of aclsparseSpMMOp (ALG1) with the reference perf test's byte and
    flop model (spmm_op_perf.cpp:325-360)."""
    from ops_sparse.spmm import SpMMOp

    cfg = case
    op = SpMMOp(cfg["m"], cfg["k"], cfg["rp"], cfg["col"], cfg["val"], cfg["b"], cfg["c"])
    stream = torch.cuda.current_stream()
    sink = torch.empty((), dtype=torch.float32, device=flush_buf.device)
    for _ in range(warmup):
        op.run(cfg["b"], cfg["c"], cfg["alpha"], cfg["beta"])
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        if cfg["flush"]:
            torch.sum(flush_buf, dim=0, out=sink)
        a.record(stream)
        op.run(cfg["b"], cfg["c"], cfg["alpha"], cfg["beta"])
        b.record(stream)
    torch.cuda.synchronize()
    t = statistics.median(sorted(a.elapsed_time(b) for a, b in evs))
    op.close()
    nnz, m, k, n = cfg["col"].numel(), cfg["m"], cfg["k"], cfg["n"]
    elem = cfg["val"].element_size()
    nbytes = nnz * elem + nnz * 4 + (m + 1) * 4 + k * n * elem + (m * n * elem if cfg["beta"] != 0 else 0) + m * n * elem
    fl = 2.0 * nnz * n + 2.0 * m * n
    return dict(m=m, k=k, n=n, nnz=nnz, dtype=str(cfg["val"].dtype).split(".")[-1], median_ms=t,
                algorithmic_bytes=nbytes, gbs=nbytes / (t * 1e-3) / 1e9, frac=nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS,
                gflops=fl / (t * 1e-3) / 1e9, l2_mall_flushed=cfg["flush"])


def cpu_baseline(w, seconds):
    """Single-threaded oracle SpMV (the reference host golden restated in C) on a bounded sample:
    whole SpMVs of the headline matrix, repeated for about ``seconds``.  fp32 workloads use
    oracle_spmv_f64 (SpmvCpu<float>: fp64 accumulation), fp16/bf16 ones oracle_spmv_lowp
    (SpmvCpu<float, half|bf16>: fp32 accumulation, one rounding to the output type)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np
    import oracle
    from ops_sparse.workloads import algorithmic_bytes

    host = w.to("cpu")
    rp = host.row_ptr.numpy().astype(np.int64)
    lowp = w.values.dtype in (torch.float16, torch.bfloat16)
    if lowp:
        kind = oracle.K_F16 if w.values.dtype == torch.float16 else oracle.K_BF16
        bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
        args = (rp, host.col_ind.numpy(), bits(host.values), bits(host.x), bits(host.y0.to(w.out_dtype)))
        serial = lambda: oracle.spmv_lowp(*args, kind, kind, w.alpha, w.beta)  # noqa: E731
        par = lambda t: oracle.spmv_lowp_threads(*args, kind, kind, w.alpha, w.beta, t)  # noqa: E731
        fn_name = "oracle_spmv_lowp (fp32 accumulation, one RNE rounding)"
    else:
        args = (rp, host.col_ind.numpy(), host.values.numpy(), host.x.numpy(), host.y0.numpy())
        serial = lambda: oracle.spmv_f64(*args, w.alpha, w.beta)  # noqa: E731
        par = lambda t: oracle.spmv_f64_threads(*args, w.alpha, w.beta, t)  # noqa: E731
        fn_name = "oracle_spmv_f64 (fp64 accumulation)"
    serial()  # page the arrays in
    n, t0 = 0, time.perf_counter()
    while True:
        serial()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / n
    # this build's row-parallel restatement on all host cores, labelled as such
    # (the GPU box's CPU share is 16 cores, whatever the machine shows)
    threads = min(len(os.sched_getaffinity(0)), 16)
    m, t0 = 0, time.perf_counter()
    while True:
        par(threads)
        m += 1
        el2 = time.perf_counter() - t0
        if el2 >= seconds / 2:
            break
    per2 = el2 / m
    parallel = {"value": algorithmic_bytes(w) / per2 / 1e9, "unit": "GB/s", "cores": threads,
                "kind": "port, row-parallel (this build's restatement, not the reference's serial golden)",
                "ms_per_spmv": per2 * 1e3, "sample": f"{m} full SpMVs in {el2:.1f} s"}
    return {"value": algorithmic_bytes(w) / per / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "parallel": parallel,
            "ms_per_spmv": per * 1e3, "gflops": 2 * w.nnz / per / 1e9,
            "sample": f"{n} full SpMVs of the headline matrix {w.name} ({w.rows} rows, {w.nnz} nnz) in {el:.1f} s, "
                      f"oracle/spmv_oracle.c {fn_name}, 1 thread",
            "cpu": cpu_model(), "host_nproc": os.cpu_count()}


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), else the machine type."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


NARROW_PATH = "row kernels, narrow columns"
ALG1_CONFIGS = ("c1", "c2", "c3", "c4h", "c5")  # also measured on CSR_ALG1's reference-sized workspace
LINE_RATE = 64e9  # 128-byte lines per second from the MALL (random x gathers), measured on MI355X


def ceilings(w, nbytes, path):
    """Lower bounds on one SpMV's time (ms): algorithmic bytes at 8 TB/s; one
    MALL line per x gather at the measured line rate (the bound of gathering
    x straight from memory when x exceeds an XCD's L2); and, on the staged
    path, its own design traffic at 8 TB/s; on the narrow-column row kernel,
    its bytes (2-byte instead of 4-byte column indices) at 8 TB/s."""
    from ops_sparse.workloads import staged_bytes

    c = {"algorithmic_hbm": nbytes / (HBM_PEAK_GBS * 1e6), "random_line_gathers": w.nnz / LINE_RATE * 1e3}
    if path == "staged gather":
        c["staged_traffic_hbm"] = staged_bytes(w) / (HBM_PEAK_GBS * 1e6)
    if path == NARROW_PATH:
        c["narrow_traffic_hbm"] = (nbytes - 2 * w.nnz) / (HBM_PEAK_GBS * 1e6)
    return c


def load_traffic(name):
    path = os.path.join(REPO, "profiles", f"traffic_{name}.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the SpMV path runs on one device (rows would shard by nnz-balanced ranges with x all-gathered)", file=sys.stderr)
        sys.exit(2)
    from ops_sparse.workloads import algorithmic_bytes, flops

    if args.profile:
        profile_mode(args.profile, args.steps)
        return
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    flush_buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
    names = [HEADLINE] if args.only_headline else [n.strip() for n in args.configs.split(",") if n.strip()]
    if HEADLINE not in names:
        names.append(HEADLINE)
    # c2 first when measured: the first SpMV of the process also pays for
    # loading the code objects (and c2's variants reuse its matrix)
    names = [n for n in names if n == "c2"] + [n for n in names if n != "c2"]
    # load the code objects before anything is timed: one small SpMV
    from ops_sparse import workloads as wl_warm
    warm_w = wl_warm.laplacian_2d(n=256, device=dev)
    measure(warm_w, 2, 1, flush_buf)
    del warm_w
    results, headline_w, headline = {}, None, None
    for name in names:
        w = make(name, dev)
        torch.cuda.synchronize()
        m = measure(w, args.steps, args.warmup, flush_buf)
        nbytes = algorithmic_bytes(w)
        gbs = nbytes / (m["median_ms"] * 1e-3) / 1e9
        r = dict(workload=w.name, rows=w.rows, nnz=w.nnz, op=w.trans, dtype=str(w.values.dtype).split(".")[-1],
                 algorithmic_bytes=nbytes, gbs=gbs, frac=gbs / HBM_PEAK_GBS,
                 gflops=flops(w) / (m["median_ms"] * 1e-3) / 1e9,
                 warm_gbs=nbytes / (m["warm_ms"] * 1e-3) / 1e9, **m)
        r["workspace_per_algorithmic_byte"] = m["workspace_bytes"] / nbytes
        r["ceilings_ms"] = ceilings(w, nbytes, m["path"])
        bound_key = {"staged gather": "staged_traffic_hbm", NARROW_PATH: "narrow_traffic_hbm"}.get(
            m["path"], "algorithmic_hbm")
        r["bound"] = {"staged_traffic_hbm": "staged traffic at 8 TB/s",
                      "narrow_traffic_hbm": "narrow-column traffic at 8 TB/s"}.get(bound_key, "hbm")
        r["frac_of_bound"] = r["ceilings_ms"][bound_key] / m["median_ms"]
        if name == "c1":
            r["graph_ms"] = graph_ms(w)
            r["graph_gbs"] = nbytes / (r["graph_ms"] * 1e-3) / 1e9
        print(f"# {name}: {json.dumps(r)}", file=sys.stderr, flush=True)
        results[name] = r
        if name in ALG1_CONFIGS and not args.only_headline:
            # the same matrix on CSR_ALG1's reference-sized workspace (row
            # kernels; atomic scatter for opA = T)
            from ops_sparse._lib import SpMVAlg
            ma = measure(w, args.steps, args.warmup, flush_buf, alg=SpMVAlg.CSR_ALG1)
            ra = dict(workload=w.name + " (CSR_ALG1)", rows=w.rows, nnz=w.nnz, op=w.trans, algorithmic_bytes=nbytes,
                      median_ms=ma["median_ms"], gbs=nbytes / (ma["median_ms"] * 1e-3) / 1e9,
                      frac=nbytes / (ma["median_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, preprocess_ms=ma["preprocess_ms"],
                      workspace_bytes=ma["workspace_bytes"],
                      workspace_per_algorithmic_byte=ma["workspace_bytes"] / nbytes)
            print(f"# {name}_alg1: {json.dumps(ra)}", file=sys.stderr, flush=True)
            results[name + "_alg1"] = ra
        if name == HEADLINE:
            headline_w, headline = w, r
            cpu = None if args.no_cpu_baseline else cpu_baseline(headline_w, args.cpu_seconds)
        if name == "c2":
            if not args.only_headline:
                for key, v in dtype_variants(w).items():
                    mv = measure(v, args.steps, args.warmup, flush_buf)
                    vb = algorithmic_bytes(v)
                    results[key] = dict(workload=v.name, rows=v.rows, nnz=v.nnz, op=v.trans,
                                        dtype=str(v.values.dtype).split(".")[-1], algorithmic_bytes=vb,
                                        gbs=vb / (mv["median_ms"] * 1e-3) / 1e9,
                                        frac=vb / (mv["median_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                        median_ms=mv["median_ms"], p90_ms=mv["p90_ms"], warm_ms=mv["warm_ms"],
                                        preprocess_ms=mv["preprocess_ms"], workspace_bytes=mv["workspace_bytes"],
                                        workspace_per_algorithmic_byte=mv["workspace_bytes"] / vb)
                    del v
            from ops_sparse._lib import SpMVOpAlg
            for alg in (SpMVOpAlg.ALG1, SpMVOpAlg.ALG2):
                t, (setup_first, setup) = measure_spmvop(w, alg, args.steps, args.warmup, flush_buf)
                key = f"c2_spmvop_{alg.name.lower()}"
                results[key] = dict(workload=f"{w.name} through aclsparseSpMVOp {alg.name} (Z != Y)", rows=w.rows,
                                    nnz=w.nnz, op="N", dtype="float32", algorithmic_bytes=nbytes, median_ms=t,
                                    gbs=nbytes / (t * 1e-3) / 1e9, frac=nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                    create_descr_ms=setup, create_descr_first_ms=setup_first)
            for key, case in spmm_cases(dev, w):
                results[key] = measure_spmm(case, args.steps, args.warmup, flush_buf)
                print(f"# {key}: {json.dumps(results[key])}", file=sys.stderr, flush=True)
        del w
        torch.cuda.empty_cache()
    h = headline
    out = {
        "metric": METRIC,
        "value": round(h["gbs"], 2),
        "unit": "GB/s",
        "gflops": round(h["gflops"], 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["median_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "compute_dtype": "fp32",
        "data": "synthetic (seeded: 32 uniform sorted columns per row, values N(0,1), x U(-1,1), fp16)",
        "config": {"workload": h["workload"], "rows": h["rows"], "nnz": h["nnz"], "alpha": 1.0, "beta": 0.0,
                   "row_offsets": "int64", "col_ind": "int32", "values_x_y": "fp16", "op": "N",
                   "l2_mall_flushed": True, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(h["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(h["frac"], 4), "traffic": load_traffic(HEADLINE),
                     "kernel": ("StageGatherKernel + StageTileKernel + StageFixupKernel: the staged-gather SpMV "
                                "(the row kernel launched before them exits at once)"
                                if h["path"] == "staged gather" else "SpmvStreamFlatKernel"),
                     "algorithmic_bytes_per_launch": h["algorithmic_bytes"],
                     "ceilings_ms": {k: round(v, 5) for k, v in h["ceilings_ms"].items()},
                     "frac_of_path_bound": round(h["frac_of_bound"], 4)},
        "cpu_baseline": cpu,
        "configs": {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in results.items()},
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
