"""Benchmark of the MI355X verify/draft hot path.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--only a,b] [--no-cpu]

Headline (the `value`): the fused RMSNorm -> linear with fp8-e4m3 weights
and per-channel fp32 scales, x bf16 [64, 4096] (a 64-node verify tree),
W [14336, 4096], gamma, bf16 out — algorithmic GB/s of one call. A step is
one call; weights rotate over enough copies that no call reads W from the
256 MB Infinity Cache. Calls go straight through the C ABI with
preallocated outputs on torch's current stream, timed with HIP events on
that stream. Every other workload is timed in the same run into "detail"
(fp8 at M = 8 / 32, the fp32 TF32-off linear, the multi-verify chain
without and with the lm_head bias and in fp32 with the bias, the
tree-verify step, one draft step of 8 sequences over a 128256-token
vocabulary, the INT4 linear at M = 256), each with its roofline
fraction against its own bound; "verify_step_us" holds the verify steps.

Prints ONE JSON line. The CPU baselines time the oracle's eager
restatement of the headline workload and of the fp32 configuration on this
host's cores; "cpu_context" in "detail" times the same restatement of the
multi-verify, the tree-verify step and the INT4 linear (whole calls, a
median of at most three) for context.

`value` and every `us_per_call` are the W warmup + K timed steps the
command line asks for. A GPU that was idle (each case is built on the CPU
first) spends its first ~10-20 ms of work in a lower clock state, so a
short run times that ramp; each entry therefore also carries `steady_*`
figures: the same calls timed again right after a 30 ms untimed run-in of
the same work, at least 100 calls (10 for the verify calls over 1 GB of
weights; the top-level `steady_state` for the headline). They are
reported beside `value`, never in its place.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "mtp-engine_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
FP32_MFMA_PEAK_TFLOPS = 157.3
MALL_BYTES = 256 * 2 ** 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def rotations(weight_bytes: int) -> int:
    return max(2, -(-512 * 2 ** 20 // max(1, weight_bytes)) + 1)


class Case:
    """A workload bound to preallocated device buffers; launch(i) enqueues
    one kernel launch on rotation i. mfma_peak: the dense MFMA peak of the
    arithmetic the kernels run (bf16/fp16, or fp32 for the TF32-off mode)."""

    def __init__(self, name, launch, nbytes, flops, bound, nrot,
                 mfma_peak=BF16_MFMA_PEAK_TFLOPS):
        self.name, self.launch, self.nbytes, self.flops = name, launch, nbytes, flops
        self.bound, self.nrot, self.mfma_peak = bound, nrot, mfma_peak


def time_case(torch, case: Case, steps: int, warmup: int):
    for i in range(warmup):
        case.launch(i)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(st)
    for i in range(steps):
        case.launch(i)
    t1.record(st)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    return ms / steps


RUN_IN_MS = 30.0


def time_steady(torch, case: Case, steps: int, step_ms: float):
    """ms per call after an untimed run-in of RUN_IN_MS of the same calls
    (wall clock, in chunks of ~2 ms), timed like time_case."""
    chunk = max(1, int(2.0 / max(step_ms, 1e-3)))
    t0 = time.perf_counter()
    i = 0
    while (time.perf_counter() - t0) * 1e3 < RUN_IN_MS:
        for _ in range(chunk):
            case.launch(i)
            i += 1
        torch.cuda.synchronize()
    return time_case(torch, case, steps, 0)


def make_fp8_case(torch, lib, L, M: int):
    from mtp_hip import workloads
    d = workloads.fp8_linear(M)
    dev = torch.device("cuda")
    N, K = d["weight_fp8"].shape
    wbytes = N * K
    nrot = rotations(wbytes + N * 4)
    ws_list = [d["weight_fp8"].to(dev) for _ in range(nrot)]
    sc_list = [d["wscale"].to(dev) for _ in range(nrot)]
    x = d["x"].to(dev)
    gamma = d["gamma"].to(dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    nws = lib.mtp_rmsnorm_linear_workspace_bytes(L.BF16, L.FP8E4M3, M, N, K)
    ws = torch.zeros(max(nws, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.mtp_fused_rmsnorm_linear_fp8
    args = [(x.data_ptr(), L.BF16, M, K, w.data_ptr(), L.FP8E4M3, s.data_ptr(), N, None, 0,
             gamma.data_ptr(), L.F32, ctypes.c_float(d["eps"]), 1, y.data_ptr(), ws.data_ptr(),
             nws, stream) for w, s in zip(ws_list, sc_list)]

    def launch(i):
        st = fn(*args[i % nrot])
        if st != 0:
            raise RuntimeError(f"fp8 launch failed: {st}")

    nbytes = M * K * 2 + N * K + N * 4 + K * 4 + M * N * 2
    flops = 2 * M * N * K
    case = Case(f"fp8_rmsnorm_linear_M{M}", launch, nbytes, flops, "hbm", nrot)
    case.keep = (ws_list, sc_list, x, gamma, y, ws, d)
    return case


def make_fp32_case(torch, lib, L, M=16, K=1024, N=4096):
    """fp32 RMSNorm+linear (TF32 off); the default is the fp32 configuration,
    M=8, K=4096 the MTP head's shape (opt-in with --only fp32_M8_K4096)."""
    from mtp_hip import workloads
    d = workloads.fp32_linear(M=M, K=K, N=N)
    dev = torch.device("cuda")
    M, K = d["x"].shape
    N = d["weight"].shape[0]
    nrot = rotations(N * K * 4)
    wl = [d["weight"].to(dev) for _ in range(nrot)]
    x, gamma = d["x"].to(dev), d["gamma"].to(dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    nws = lib.mtp_rmsnorm_linear_workspace_bytes(L.F32, L.F32, M, N, K)
    ws = torch.zeros(max(nws, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.mtp_fused_rmsnorm_linear
    args = [(x.data_ptr(), L.F32, M, K, w.data_ptr(), L.F32, N, None, 0, gamma.data_ptr(), L.F32,
             ctypes.c_float(d["eps"]), ctypes.c_float(1.0), 1, y.data_ptr(), ws.data_ptr(), nws,
             stream) for w in wl]

    def launch(i):
        st = fn(*args[i % nrot])
        if st != 0:
            raise RuntimeError(f"fp32 launch failed: {st}")

    nbytes = M * K * 4 + N * K * 4 + K * 4 + M * N * 4
    case = Case(f"fp32_rmsnorm_linear_M{M}_K{K}_N{N}", launch, nbytes, 2 * M * N * K, "hbm", nrot,
                FP32_MFMA_PEAK_TFLOPS)
    case.keep = (wl, x, gamma, y, ws)
    return case


def make_int4_case(torch, lib, L):
    """INT4 weight-only RMSNorm+linear, x bf16 [256, 8192], W [28672, 8192]
    group 128 with fp16 scales, gamma, bf16 out (one launch = the prologue
    that writes the fp16 activations plus the MFMA GEMM)."""
    from mtp_hip import workloads
    d = workloads.int4_linear()
    dev = torch.device("cuda")
    M, K = d["x"].shape
    N = d["packed"].shape[0]
    group = d["group"]
    wbytes = N * K // 2 + d["scales"].numel() * 2
    nrot = rotations(wbytes)
    pl = [d["packed"].to(dev) for _ in range(nrot)]
    sl = [d["scales"].to(dev) for _ in range(nrot)]
    x, gamma = d["x"].to(dev), d["gamma"].to(dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    nws = lib.mtp_rmsnorm_linear_workspace_bytes(L.BF16, L.U8, M, N, K)
    ws = torch.zeros(max(nws, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.mtp_fused_int4_matmul
    args = [(x.data_ptr(), L.BF16, M, K, p.data_ptr(), s.data_ptr(), L.F16, N, group,
             L.NIBBLE_OFFSET8, gamma.data_ptr(), L.F32, ctypes.c_float(d["eps"]), 1,
             y.data_ptr(), ws.data_ptr(), nws, stream) for p, s in zip(pl, sl)]

    def launch(i):
        st = fn(*args[i % nrot])
        if st != 0:
            raise RuntimeError(f"int4 launch failed: {st}")

    nbytes = M * K * 2 + wbytes + K * 4 + M * N * 2
    case = Case(f"int4_rmsnorm_linear_M{M}", launch, nbytes, 2 * M * N * K, "mfma", nrot)
    case.keep = (pl, sl, x, gamma, y, ws)
    return case


def make_verify_case(torch, lib, L, dtype=None, bias=False):
    """fused_multi_verify at the multi-verify workload's shape: hidden [8, 5,
    4096], lm_head [128256, 4096], optionally with the lm_head's bias [128256]
    (the engine's call, mtp_engine.py:1237-1242), in bf16 or in the engine's
    default fp32."""
    import torch.nn.functional as F
    from mtp_hip import workloads
    dtype = dtype or torch.bfloat16
    d = workloads.multi_verify(dtype=dtype, bias=bias)
    dev = torch.device("cuda")
    hidden = d["hidden"].to(dev)
    W = d["weight"].to(dev)
    b = d["bias"].to(dev) if bias else None
    B, S, K = hidden.shape
    V = W.shape[0]
    D = S - 1
    esz = hidden.element_size()
    # drafts from the target argmax (synthetic input construction only)
    with torch.no_grad():
        Wf = W.float().contiguous()
        top = F.linear(hidden.reshape(-1, K).float(), Wf, None if b is None else b.float())
        top = top.argmax(-1)
        del Wf
    draft = workloads.make_chain_drafts(top.reshape(B, S).cpu(), V, d["seed"]).to(dev)
    draft32 = draft.to(torch.int32)
    accept = torch.empty((B, D), dtype=torch.int8, device=dev)
    acc_n = torch.empty((B,), dtype=torch.int32, device=dev)
    corr = torch.empty((B,), dtype=torch.int32, device=dev)
    code = L.code(dtype)
    nws = lib.mtp_verify_workspace_bytes(code, B * S, S, V, K)
    ws = torch.zeros(nws, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.mtp_fused_multi_verify
    args = (hidden.data_ptr(), code, B, S, K, W.data_ptr(), code, V,
            None if b is None else b.data_ptr(), code if bias else 0,
            draft32.data_ptr(), D, accept.data_ptr(), acc_n.data_ptr(), corr.data_ptr(), None,
            ws.data_ptr(), nws, stream)

    def launch(i):
        st = fn(*args)
        if st != 0:
            raise RuntimeError(f"multi-verify launch failed: {st}")

    nbytes = B * S * K * esz + V * K * esz + (V * esz if bias else 0) + B * D * 4 + B * D + \
        B * 4 * 2
    name = "multi_verify_B8_S5_V128256" + ("_bias" if bias else "") + \
        ("_fp32" if dtype == torch.float32 else "")
    peak = FP32_MFMA_PEAK_TFLOPS if dtype == torch.float32 else BF16_MFMA_PEAK_TFLOPS
    case = Case(name, launch, nbytes, 2 * B * S * K * V, "hbm", 1, peak)
    case.keep = (hidden, W, b, draft32, accept, acc_n, corr, ws)
    return case


def make_tree_verify_case(torch, lib, L):
    """Tree-verify step: 64-node attention over 2048 paged context tokens plus
    the ancestors (one launch), then RMSNorm+linear 4096 -> 4096 bf16."""
    import math
    from mtp_hip import workloads
    d = workloads.tree_verify()
    dev = torch.device("cuda")
    t = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
    N, H, D = d["q"].shape
    Lc = d["page_table"].shape[-1]
    P = d["k_pages"].shape[0]
    ps = d["page_size"]
    tmask = t["tree_mask"].contiguous()
    att = torch.empty_like(t["q"])
    K = H * D
    Nout = d["weight"].shape[0]
    # weights and the paged KV cache both rotate past the MALL
    nrot = rotations(min(Nout * K * 2, 2 * P * H * ps * D * 2))
    wl = [t["weight"]] + [t["weight"].clone() for _ in range(nrot - 1)]
    kpl = [t["k_pages"]] + [t["k_pages"].clone() for _ in range(nrot - 1)]
    vpl = [t["v_pages"]] + [t["v_pages"].clone() for _ in range(nrot - 1)]
    y = torch.empty((N, Nout), dtype=torch.bfloat16, device=dev)
    na = lib.mtp_attention_workspace_bytes(L.BF16, 1, N, H, D, Lc, N)
    nl = lib.mtp_rmsnorm_linear_workspace_bytes(L.BF16, L.BF16, N, Nout, K)
    ws = torch.zeros(max(na, nl, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    scale = ctypes.c_float(1.0 / math.sqrt(D))
    a_args = [(t["q"].data_ptr(), L.BF16, N, H, D, kp.data_ptr(), vp.data_ptr(), P,
               t["page_table"].data_ptr(), Lc, ps, t["k_tree"].data_ptr(), t["v_tree"].data_ptr(),
               tmask.data_ptr(), L.F32, scale, att.data_ptr(), ws.data_ptr(), na, stream)
              for kp, vp in zip(kpl, vpl)]
    l_args = [(att.data_ptr(), L.BF16, N, K, w.data_ptr(), L.BF16, Nout, None, 0, None, 0,
               ctypes.c_float(d["eps"]), ctypes.c_float(1.0), 1, y.data_ptr(), ws.data_ptr(), nl,
               stream) for w in wl]

    def launch(i):
        st = lib.mtp_tree_verify_attention(*a_args[i % nrot])
        if st != 0:
            raise RuntimeError(f"tree-verify attention failed: {st}")
        st = lib.mtp_fused_rmsnorm_linear(*l_args[i % nrot])
        if st != 0:
            raise RuntimeError(f"tree-verify linear failed: {st}")

    # bytes: context KV + tree KV + q + out + table + mask, then the linear
    att_bytes = 2 * Lc * H * D * 2 + 2 * N * H * D * 2 + 2 * N * H * D * 2 + Lc * 4 + N * N * 4
    lin_bytes = N * K * 2 + Nout * K * 2 + N * Nout * 2
    flops = 4 * H * D * (N * Lc + int(d["tree_mask"].sum())) + 2 * N * Nout * K
    case = Case("tree_verify_step_64nodes_ctx2048", launch, att_bytes + lin_bytes, flops, "hbm", nrot)
    case.keep = (t, tmask, att, wl, kpl, vpl, y, ws)
    return case


def make_draft_step_case(torch, lib, L, B=8, K=4096, V=128256):
    """One on-device draft step of B sequences (the draft chain around the
    head GEMM, mtp_engine.py:735-777): RMSNorm of the hidden rows, RMSNorm ->
    linear onto the vocabulary (bf16 head [V, K] with bias), greedy argmax
    with the embedding gather of the chosen tokens, and the combine-norm of
    the normed hidden plus the embeddings (add + RMSNorm). Bound by reading
    the head weights once."""
    from mtp_hip import ops
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(11)  # seeded on the device: 2 x 1 GB of draws
    dt = torch.bfloat16
    hidden = torch.randn(B, K, generator=g, device=dev).to(dt)
    nrot = rotations(V * K * 2)
    wl = [(0.02 * torch.randn(V, K, generator=g, device=dev)).to(dt)]
    wl += [wl[0].clone() for _ in range(nrot - 1)]
    bias = (0.1 * torch.randn(V, generator=g, device=dev)).to(dt)
    head_w = (1 + 0.1 * torch.randn(K, generator=g, device=dev)).to(dt)
    comb_w = (1 + 0.1 * torch.randn(K, generator=g, device=dev)).to(dt)
    table = torch.randn(V, K, generator=g, device=dev).to(dt)

    def launch(i):
        h_norm = ops.rmsnorm(hidden, head_w, 1e-6)
        logits = ops.rmsnorm_linear(hidden, wl[i % nrot], bias, 1e-6)
        _, emb = ops.argmax(logits, table)
        ops.rmsnorm(h_norm, comb_w, 1e-6, residual=emb)

    # head weights and bias once, the logits written and read back, the
    # hidden rows (three reads), the gathered embeddings, two outputs
    nbytes = V * K * 2 + V * 2 + 2 * B * V * 2 + 7 * B * K * 2 + 2 * K * 2
    case = Case(f"draft_step_B{B}_K{K}_V{V}", launch, nbytes, 2 * B * V * K, "hbm", nrot)
    case.keep = (hidden, wl, bias, head_w, comb_w, table)
    return case


def pmc_traffic(name: str):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor),
    or None when no summary is committed."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            d = json.load(f)
        return int(d["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _time_cpu(fn, seconds):
    fn()
    times = []
    t_end = time.time() + seconds
    while len(times) < 5 or (time.time() < t_end and len(times) < 20000):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times), len(times)


def cpu_baseline_fp32(torch):
    """The fp32 RMSNorm+linear configuration (x [16,1024], W [4096,1024],
    gamma, TF32 off) through the oracle's eager restatement, whole calls."""
    from mtp_hip import workloads
    from oracle import eager as O
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    d = workloads.fp32_linear()
    fn = lambda: O.rmsnorm_linear(d["x"], d["weight"], None, d["eps"], 1.0, gamma=d["gamma"])
    med, n = _time_cpu(fn, 5.0)
    M, K = d["x"].shape
    N = d["weight"].shape[0]
    nbytes = M * K * 4 + N * K * 4 + K * 4 + M * N * 4
    return dict(value=round(nbytes / med / 1e9, 3), unit="GB/s", us_per_call=round(med * 1e6, 1),
                cores=torch.get_num_threads(), kind="port",
                sample=f"full fp32 workload, median of {n} calls; {_cpu_model()}")


def cpu_baseline_fp8(torch, M: int):
    from mtp_hip import workloads
    from oracle import eager as O
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    d = workloads.fp8_linear(M)
    fn = lambda: O.rmsnorm_linear_fp8(d["x"], d["weight_fp8"], d["wscale"], None, d["eps"],
                                      gamma=d["gamma"])
    # a bounded sample: repeated full calls for about 10 s of CPU work
    med, n = _time_cpu(fn, 10.0)
    N, K = d["weight_fp8"].shape
    nbytes = M * K * 2 + N * K + N * 4 + K * 4 + M * N * 2
    return dict(value=round(nbytes / med / 1e9, 3), unit="GB/s", cores=torch.get_num_threads(),
                kind="port",
                sample=f"full workload (M={M}), median of {n} runs, "
                       f"{med * 1e3:.1f} ms/run; eager fp32 restatement (fp8 decode + F.linear); "
                       f"{_cpu_model()}")


def cpu_context(torch, seconds: float = 8.0):
    """The oracle's eager restatement of the other workloads, on the host
    cores, for context: multi-verify (B = 8, depth 4, V = 128256 bf16 head,
    the B x D loop of logits and argmax), the tree-verify step (64-node
    attention over 2048 paged tokens, then RMSNorm -> linear 4096 -> 4096)
    and the INT4 RMSNorm+linear (M = 256, the reference's per-group dequant
    loop, then fp32 F.linear). Each: one untimed call, then whole calls
    until `seconds` have passed (at least one, at most three), median."""
    import math
    from mtp_hip import workloads
    from oracle import eager as O
    torch.set_num_threads(len(os.sched_getaffinity(0)))

    def timed(fn):
        fn()
        times = []
        t_end = time.time() + seconds
        while not times or (time.time() < t_end and len(times) < 3):
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
        return round(statistics.median(times) * 1e6, 1), len(times)

    out = {}
    d = workloads.multi_verify()
    B, D = d["B"], d["D"]
    V = d["weight"].shape[0]
    g = torch.Generator().manual_seed(d["seed"])
    draft = torch.randint(0, V, (B, D), generator=g, dtype=torch.int32)
    us, n = timed(lambda: O.fused_multi_verify(d["hidden"], d["weight"], draft))
    out["multi_verify"] = dict(us_per_call=us, runs=n)
    del d
    d = workloads.tree_verify()
    scale = 1.0 / math.sqrt(d["q"].shape[-1])

    def tree_step():
        att = O.tree_verify_attention(d["q"], d["k_pages"], d["v_pages"], d["page_table"],
                                      d["page_size"], d["k_tree"], d["v_tree"], d["tree_mask"],
                                      scale)
        return O.rmsnorm_linear(att.reshape(att.shape[0], -1).to(torch.bfloat16), d["weight"],
                                None, d["eps"], 1.0)
    us, n = timed(tree_step)
    out["tree_verify"] = dict(us_per_call=us, runs=n)
    del d
    d = workloads.int4_linear()
    us, n = timed(lambda: O.int4_matmul(d["x"], d["packed"], d["scales"], d["K"], d["group"],
                                        gamma=d["gamma"], norm=True, eps=d["eps"]))
    out["int4_M256"] = dict(us_per_call=us, runs=n)
    return dict(cores=torch.get_num_threads(), kind="port", workloads=out, cpu=_cpu_model())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--all", action="store_true", help="(kept for old scripts: every workload "
                    "is timed by default)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a 256 MiB device copy (known HBM bytes) so rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE can be scaled to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the library runs on a single MI355X and has no "
              "multi-GPU path (the verify kernels would shard the vocabulary columns across "
              "GPUs, one process per GPU).", file=sys.stderr)
        sys.exit(2)

    import torch
    from mtp_hip import _lib as L
    lib = L.load()
    assert torch.cuda.is_available(), "bench.py needs a HIP GPU"

    detail = {}
    headline = None
    builders = [("fp8_M64", lambda: make_fp8_case(torch, lib, L, 64)),
                ("fp8_M8", lambda: make_fp8_case(torch, lib, L, 8)),
                ("fp8_M32", lambda: make_fp8_case(torch, lib, L, 32)),
                ("fp32_M16", lambda: make_fp32_case(torch, lib, L)),
                ("multi_verify", lambda: make_verify_case(torch, lib, L)),
                ("multi_verify_bias", lambda: make_verify_case(torch, lib, L, bias=True)),
                ("multi_verify_fp32", lambda: make_verify_case(torch, lib, L, torch.float32,
                                                               bias=True)),
                ("tree_verify", lambda: make_tree_verify_case(torch, lib, L)),
                ("draft_step", lambda: make_draft_step_case(torch, lib, L)),
                ("int4_M256", lambda: make_int4_case(torch, lib, L))]
    if args.only:
        builders = [b for b in builders if b[0] in args.only.split(",")]
        if "fp32_M8_K4096" in args.only.split(","):  # opt-in: the MTP head's fp32 shape
            builders.append(("fp32_M8_K4096", lambda: make_fp32_case(torch, lib, L, 8, 4096)))
    for key, mk in builders:
        log(f"[bench] building {key}")
        case = mk()
        steps = args.steps if case.nbytes < 2e8 else max(10, args.steps // 10)
        ms = time_case(torch, case, steps, args.warmup)
        us = ms * 1e3
        gbs = case.nbytes / (ms * 1e-3) / 1e9
        tfl = case.flops / (ms * 1e-3) / 1e12
        hbm_frac = gbs / HBM_PEAK_GBS
        mfma_frac = tfl / case.mfma_peak
        frac = hbm_frac if case.bound == "hbm" else mfma_frac
        steps_st = max(steps, 100 if case.nbytes < 2e8 else 10)
        ms_st = time_steady(torch, case, steps_st, ms)
        frac_st = frac * ms / ms_st
        detail[key] = dict(workload=case.name, us_per_call=round(us, 3), GBps=round(gbs, 1),
                           TFLOPs=round(tfl, 2), bound=case.bound,
                           roofline_frac=round(frac, 4),
                           hbm_frac=round(hbm_frac, 4), mfma_frac=round(mfma_frac, 4),
                           algorithmic_bytes=case.nbytes, flops=case.flops,
                           weight_rotations=case.nrot, steps=steps,
                           steady_us_per_call=round(ms_st * 1e3, 3),
                           steady_roofline_frac=round(frac_st, 4), steady_steps=steps_st)
        log(f"[bench] {key}: {us:.2f} us  {gbs:.0f} GB/s  {tfl:.1f} TFLOP/s  "
            f"(steady {ms_st * 1e3:.2f} us)")
        if key == "fp8_M64":
            headline = (case, ms, steps, ms_st, steps_st)
        del case
        torch.cuda.empty_cache()

    if args.copy_calib:
        n = 256 * 2 ** 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        detail["copy_calib"] = dict(bytes_read=n, bytes_written=n, launches=5)
        del src, dst

    if headline is None:  # --only without the headline workload: the detail alone
        print(json.dumps({"detail": detail}), flush=True)
        return

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle, fp8 M=64)")
        cpu = cpu_baseline_fp8(torch, 64)
        log("[bench] cpu baseline (oracle, fp32 configuration)")
        detail["cpu_baseline_fp32_M16"] = cpu_baseline_fp32(torch)
        if not args.only:
            log("[bench] cpu context (oracle: multi-verify, tree-verify step, INT4)")
            detail["cpu_context"] = cpu_context(torch)
    verify_us = {k: detail[k]["us_per_call"] for k in ("multi_verify", "multi_verify_bias",
                                                       "multi_verify_fp32", "tree_verify")
                 if k in detail}

    case, ms, steps, ms_st, steps_st = headline
    gbs = case.nbytes / (ms * 1e-3) / 1e9
    gbs_st = case.nbytes / (ms_st * 1e-3) / 1e9
    out = {
        "metric": "fused RMSNorm+linear TFLOP/s & GB/s (% roofline); verify-step us, 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3-weights/bf16-act/fp32-acc",
        "data": "synthetic (seeded torch CPU generator, weights rotated x%d past the 256 MB MALL)"
                % case.nrot,
        "config": {"workload": "fused RMSNorm+linear, fp8-e4m3 weights with per-channel fp32 "
                               "scales: x bf16 [64,4096], gamma [4096], W [14336,4096], bf16 out",
                   "M": 64, "K": 4096, "N": 14336, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": pmc_traffic("fp8_rmsnorm_linear_M64.pmc.json"),
                     "algorithmic_bytes": case.nbytes},
        "steady_state": {"value": round(gbs_st, 1), "unit": "GB/s",
                         "ms_per_step": round(ms_st, 6), "frac": round(gbs_st / HBM_PEAK_GBS, 4),
                         "steps": steps_st, "run_in_ms": RUN_IN_MS,
                         "note": "the same K calls timed after an untimed run-in of the same "
                                 "work (GPU out of its idle clock state); not the value"},
        "cpu_baseline": cpu,
        "verify_step_us": verify_us,
        "detail": detail,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
