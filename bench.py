"""Benchmark of the fused causal top-K + sparse-attention forward on one MI355X.

Workload (default, BASELINE.json config 4, the metric's shape): one layer, bf16, B=1, H=8,
T=16384, head_dim=64, d_A=32, K=128, causal; inputs ~N(0,1) from a fixed seed, already
resident in HBM; q/k/v in the attention module's natural (B,T,H,D) memory viewed as
(B,H,T,D). One step = one fused_sparse_attention call (retrieval + readout, both HIP
kernels of libwayfinder_hip.so).

Prints ONE JSON line: latency (ms) as `value`, a `roofline` object for the dominant kernel
(the readout: algorithmic bytes / its HIP-event-timed duration vs 8 TB/s), a
`cpu_baseline` object (the reference's op sequence restated in PyTorch-CPU on this host,
timed on a bounded sample and scaled to the full call), and the dense causal SDPA
comparator at the same shape on the same GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "wayfinder-attention_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

CONFIGS = {
    # name: (B, H, T, D, R, K, dtype, address distribution)
    "c1": (1, 4, 2048, 64, 32, 128, torch.float32, "normal"),
    "c3": (4, 8, 4096, 64, 32, 128, torch.bfloat16, "normal"),
    "c4": (1, 8, 16384, 64, 32, 128, torch.bfloat16, "normal"),
    "c5": (1, 8, 65536, 128, 32, 256, torch.bfloat16, "student_t"),
}
HBM_PEAK_GBS = 8000.0
# dense MFMA peaks of one MI355X (TFLOP/s) for the retrieval's score tiles, by input dtype
MFMA_PEAK_TFLOPS = {torch.bfloat16: 2500.0, torch.float16: 2500.0, torch.float32: 157.3}


def algorithmic_bytes(B, H, T, D, R, K, s):
    """Bytes the path must move at minimum per call, counting one gathered K and V row per
    (query, head, neighbour): addresses + Q + gathered K/V + output + int32 indices."""
    k = min(K, T)
    addr = 2 * B * T * R * s
    readout = B * H * T * D * s + 2 * B * H * T * k * D * s + B * H * T * D * s + 4 * B * T * k
    return addr + readout, readout


def make_inputs(cfg, device, seed=1004):
    B, H, T, D, R, K, dtype, dist = cfg
    g = torch.Generator().manual_seed(seed)
    if dist == "student_t":
        def t3(*shape):
            z = torch.randn(*shape, generator=g)
            c = (torch.randn(3, *shape, generator=g) ** 2).sum(0)
            return z / torch.sqrt(c / 3)
        qa, ka = t3(B, T, R) / R ** 0.5, t3(B, T, R) / R ** 0.5
    else:
        qa, ka = torch.randn(B, T, R, generator=g), torch.randn(B, T, R, generator=g)
    qkv = [torch.randn(B, T, H, D, generator=g) for _ in range(3)]
    cpu = dict(qa=qa.to(dtype), ka=ka.to(dtype), q=qkv[0].to(dtype), k=qkv[1].to(dtype),
               v=qkv[2].to(dtype))
    dev = {n: t.to(device) for n, t in cpu.items()}
    for n in ("q", "k", "v"):      # (B,T,H,D) memory, (B,H,T,D) view
        dev[n] = dev[n].transpose(1, 2)
        cpu[n] = cpu[n].transpose(1, 2)
    return cpu, dev


def time_loop(fn, steps, warmup):
    """Average ms per call over `steps` back-to-back calls, HIP events on the current
    stream (the stream every kernel here is launched on)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def per_call_ms(fn, reps):
    """Median / min / p90 of single-call HIP-event times."""
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b))
    ts.sort()
    return statistics.median(ts), ts[0], ts[int(0.9 * (len(ts) - 1))]


def cpu_baseline(cpu, cfg, rows_readout=512):
    """The reference path restated op by op in PyTorch-CPU (oracle/torch_reference.py) on
    this host's cores: retrieval on the reference's last row block (rows T-block..T, the
    full causal prefix), readout on the last `rows_readout` query rows; each scaled to the
    whole call (retrieval by the triangular sum of the row blocks, readout by T/rows)."""
    from oracle import torch_reference as tr

    B, H, T, D, R, K, dtype, _ = cfg
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    bm = tr._row_block(T)
    blocks = [(i0, min(i0 + bm, T)) for i0 in range(0, T, bm)]
    i0, i1 = blocks[-1]
    # warm the thread pool on a tiny problem
    tr.row_blocked_topk(cpu["qa"][:, :256], cpu["ka"][:, :256], K)
    t0 = time.perf_counter()
    idx = tr.row_blocked_topk(cpu["qa"], cpu["ka"], K, row_range=(i0, i1))
    t_ret = time.perf_counter() - t0
    ret_scale = sum((b1 - b0) * b1 for b0, b1 in blocks) / ((i1 - i0) * i1)
    r0 = T - rows_readout
    q = cpu["q"][:, :, r0:]
    sub_idx = idx[:, r0:]
    # gather on the full k/v, readout rows [r0, T) only
    t0 = time.perf_counter()
    tr.sparse_meat_reference(q, cpu["k"], cpu["v"], sub_idx, D ** -0.5)
    t_read = time.perf_counter() - t0
    total_ms = (t_ret * ret_scale + t_read * T / rows_readout) * 1e3
    return {
        "value": round(total_ms, 2), "unit": "ms", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"torch-CPU restatement of the reference path; retrieval timed on row block "
                   f"[{i0},{i1}) x{ret_scale:.3f} ({t_ret * 1e3:.0f} ms), readout on rows "
                   f"[{r0},{T}) x{T // rows_readout} ({t_read * 1e3:.0f} ms); one timed run each"),
        "retrieval_ms": round(t_ret * ret_scale * 1e3, 2),
        "readout_ms": round(t_read * T / rows_readout * 1e3, 2),
        "cpu_model": _cpu_model(),
    }


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run_leg(args, dev, K, scale, readout_bytes):
    """One kernel (or a plain copy) in isolation, for rocprofv3 counter passes."""
    from routing_attention.kernels import causal_topk, sparse_meat_attention

    if args.leg == "copy":
        src = torch.empty(128 * 2 ** 20, dtype=torch.bfloat16, device=dev["q"].device).normal_()
        dst = torch.empty_like(src)
        ms = time_loop(lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"leg": "copy", "bytes_read": src.numel() * 2,
                          "bytes_written": dst.numel() * 2, "ms": round(ms, 4)}), flush=True)
        return
    if args.leg == "topk":
        fn = lambda: causal_topk(dev["qa"], dev["ka"], K)  # noqa: E731
        ms = time_loop(fn, args.steps, args.warmup)
        print(json.dumps({"leg": "topk", "ms": round(ms, 4)}), flush=True)
        return
    idx = causal_topk(dev["qa"], dev["ka"], K)
    if args.leg == "backward":
        from routing_attention.kernels.sparse_autograd import readout_bwd, readout_fwd_lse

        out, lse2 = readout_fwd_lse(dev["q"], dev["k"], dev["v"], idx, scale)
        dout = torch.randn_like(out)
        fn = lambda: readout_bwd(dev["q"], dev["k"], dev["v"], idx, lse2, dout, scale)  # noqa: E731
        ms = time_loop(fn, args.steps, args.warmup)
        fwd_ms = time_loop(lambda: readout_fwd_lse(dev["q"], dev["k"], dev["v"], idx, scale),
                           args.steps, args.warmup)
        print(json.dumps({"leg": "backward", "ms": round(ms, 4), "fwd_lse_ms": round(fwd_ms, 4),
                          "gathered_gbs": round(2 * (readout_bytes) / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return
    fn = lambda: sparse_meat_attention(dev["q"], dev["k"], dev["v"], idx, scale)  # noqa: E731
    ms = time_loop(fn, args.steps, args.warmup)
    print(json.dumps({"leg": "readout", "ms": round(ms, 4),
                      "algorithmic_gbs": round(readout_bytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


C2 = dict(vocab=128, d_model=256, n_layers=4, n_heads=4, d_ff=1024, T=2048, B=8, K=128)


def bench_decoder(args):
    """Config 2: the 4-layer learned-address decoder forward in bf16 (random init, tokens
    uniform over the vocabulary from a seed), every layer on the fused HIP path. One step =
    one full forward (embeddings, 4 blocks, tied LM head, loss). The comparator runs the
    same blocks with dense causal SDPA attention."""
    from routing_attention.models import TransformerLM

    c = C2
    dev = torch.device("cuda:0")
    torch.manual_seed(2002)
    model = TransformerLM(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["d_ff"], c["T"],
                          dropout=0.0, attention_type="learned_address", routing_top_k=c["K"],
                          retrieval_config={"use_fused_sparse": True})
    model = model.eval().to(device=dev, dtype=torch.bfloat16)
    ids = torch.randint(0, c["vocab"], (c["B"], c["T"]),
                        generator=torch.Generator().manual_seed(3002)).to(dev)
    dense = TransformerLM(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["d_ff"], c["T"],
                          dropout=0.0, attention_type="dense").eval().to(device=dev, dtype=torch.bfloat16)

    def step():
        with torch.no_grad():
            return model(ids)

    def dense_step():
        with torch.no_grad():
            pos = torch.arange(c["T"], device=dev).unsqueeze(0)
            x = dense.token_emb(ids) + dense.pos_emb(pos)
            for blk in dense.blocks:
                x = blk(x, attn_mask=None)      # causal SDPA (is_causal=True)
            return dense.lm_head(dense.ln_f(x))

    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    ms = time_loop(step, args.steps, args.warmup)
    peak_mb = (torch.cuda.max_memory_allocated() - base) / 2 ** 20
    med, mn, p90 = per_call_ms(step, max(10, args.steps // 2))
    # the same forward captured once as a HIP graph and replayed (serving loops): the
    # launches of the ~60 kernels per forward go out as one graph launch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    gms = time_loop(graph.replay, args.steps, args.warmup)
    dms = time_loop(dense_step, args.steps, args.warmup)
    dgraph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        dense_step()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(dgraph):
        dense_step()
    dgms = time_loop(dgraph.replay, args.steps, args.warmup)
    tokens = c["B"] * c["T"]
    line = {
        "metric": "config-2 4-layer learned-address decoder forward throughput (tokens/s)",
        "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights, tokens uniform over the vocabulary from a seed)",
        "config": {"workload": "config 2: 4-layer decoder forward", **c,
                   "attention": "learned_address, fused HIP top-K + readout", "parallelism": "single GPU"},
        "latency_ms": {"mean": round(ms, 4), "median": round(med, 4), "min": round(mn, 4),
                       "p90": round(p90, 4)},
        "peak_mb": round(peak_mb, 1),
        "graph_replay_ms_per_step": round(gms, 4),
        "graph_replay_tokens_per_s": round(tokens / (gms * 1e-3), 1),
        "dense_causal_sdpa_decoder_ms": round(dms, 4),
        "dense_graph_replay_ms": round(dgms, 4),
        "vs_dense": round(dms / ms, 3),
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS) + ["c2"],
                    help="c4 (default) is the metric's workload; c2 times the 4-layer decoder")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense SDPA comparator")
    ap.add_argument("--leg", default="all", choices=["all", "topk", "readout", "backward", "copy"],
                    help="profiling aid: run only one kernel (or a 256 MiB device copy used to "
                         "calibrate the FETCH_SIZE / WRITE_SIZE counters) and print its timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this path has no multi-GPU code "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    if args.config == "c2":
        bench_decoder(args)
        return

    from routing_attention.kernels import causal_topk, fused_sparse_attention, sparse_meat_attention

    cfg = CONFIGS[args.config]
    B, H, T, D, R, K, dtype, dist = cfg
    device = torch.device("cuda:0")
    cpu, dev = make_inputs(cfg, device)
    scale = D ** -0.5
    s = torch.tensor([], dtype=dtype).element_size()
    path_bytes, readout_bytes = algorithmic_bytes(B, H, T, D, R, K, s)

    def step():
        return fused_sparse_attention(dev["qa"], dev["ka"], dev["q"], dev["k"], dev["v"], K, scale)

    if args.leg != "all":
        run_leg(args, dev, K, scale, readout_bytes)
        return

    torch.cuda.reset_peak_memory_stats()
    base_mem = torch.cuda.memory_allocated()
    _, idx = step()
    torch.cuda.synchronize()
    ms = time_loop(step, args.steps, args.warmup)
    peak_mb = (torch.cuda.max_memory_allocated() - base_mem) / 2 ** 20
    med, mn, p90 = per_call_ms(step, max(10, args.steps // 2))

    # per-kernel legs (same kernels as inside the fused call)
    ms_topk = time_loop(lambda: causal_topk(dev["qa"], dev["ka"], K), args.steps, 3)
    ms_read = time_loop(lambda: sparse_meat_attention(dev["q"], dev["k"], dev["v"], idx, scale),
                        args.steps, 3)
    read_gbs = readout_bytes / (ms_read * 1e-3) / 1e9
    score_flops = B * R * T * (T + 1)

    dense = None
    if not args.no_dense:
        qd, kd, vd = dev["q"], dev["k"], dev["v"]
        torch.cuda.reset_peak_memory_stats()
        m0 = torch.cuda.memory_allocated()
        fn = lambda: F.scaled_dot_product_attention(qd, kd, vd, is_causal=True, scale=scale)  # noqa: E731
        fn()
        torch.cuda.synchronize()
        dmed, dmin, dp90 = per_call_ms(fn, 50)
        dense = {"median_ms": round(dmed, 4), "min_ms": round(dmin, 4), "p90_ms": round(dp90, 4),
                 "peak_mb": round((torch.cuda.max_memory_allocated() - m0) / 2 ** 20, 1)}

    traffic = None
    tf = os.path.join(ROOT, "profiles", f"readout_traffic_{args.config}.json")
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("hbm_bytes_per_launch")

    line = {
        "metric": "fused top-K128+sparse-attn fwd latency (ms) @T=16384; % HBM roofline",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype],
        "data": f"synthetic ({dist} inputs from a fixed seed, resident in HBM)",
        "config": {"workload": f"fused causal top-K + sparse attention fwd, config {args.config[1:]}",
                   "B": B, "H": H, "T": T, "head_dim": D, "d_A": R, "top_k": K,
                   "qkv_memory": "(B,T,H,D)", "parallelism": "single GPU"},
        "latency_ms": {"mean": round(ms, 4), "median": round(med, 4), "min": round(mn, 4),
                       "p90": round(p90, 4)},
        "rows_per_s": round(B * T / (ms * 1e-3), 1),
        "kernels_ms": {"causal_topk": round(ms_topk, 4), "sparse_readout": round(ms_read, 4)},
        "roofline": {"bound": "hbm", "kernel": "sparse_readout_fast",
                     "achieved": round(read_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(read_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": readout_bytes},
        "path_roofline": {"algorithmic_bytes": path_bytes,
                          "achieved_gbs": round(path_bytes / (ms * 1e-3) / 1e9, 1),
                          "frac": round(path_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        # the retrieval's score contraction (q_addr . k_addr over the causal triangle,
        # B*d_A*T*(T+1) flops) against the dense MFMA peak: it is far from that bound
        "retrieval_mfma": {"kernel": "causal_topk_kernel", "flops": score_flops,
                           "achieved": round(score_flops / (ms_topk * 1e-3) / 1e12, 2),
                           "peak": MFMA_PEAK_TFLOPS[dtype], "unit": "TFLOP/s",
                           "frac": round(score_flops / (ms_topk * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS[dtype], 5)},
        "peak_mb": round(peak_mb, 1),
        "dense_causal_sdpa": dense,
        "vs_dense": round(dense["median_ms"] / med, 3) if dense else None,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cpu, cfg)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
