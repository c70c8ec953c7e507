"""Benchmark: bs=1 greedy decode of a Qwen2.5-1.5B-shaped decoder on one MI355X.

Workload: 28 layers, hidden 1536, 12 query / 2 KV heads,
head_dim 128, intermediate 8960, vocab 151936, tied embeddings, random-init bf16
N(0, 0.02) weights (RMSNorm weights ones), a 512-token prompt of uniform random ids,
256 generated tokens. One "step" = one EdgeFM.generate() call (prefill 512 + 255
graph-replayed decode steps). `value` = decode tokens/s over the K timed steps
(engine HIP events around the decode loop); prefill tokens/s is reported beside it.

Extra fields:
  roofline      the dominant decode kernel (fused post-attention RMSNorm + gate/up
                GEMV + SwiGLU, 50 % of the decode bytes) timed with HIP events around a
                graph replay of 20 x 28 launches over all 28 layers' weights, against
                8 TB/s HBM; `traffic` is read from the committed rocprofv3 --pmc summary.
  decode_loop   algorithmic bytes per decode token / measured ms per token.
  cpu_baseline  the CPU oracle (PyTorch, fp32 math on bf16 values) on this host,
                same model, a bounded sample (16-token prefill + 48 decode steps).
"""
import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "edge-fm-x_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0


def decode_bytes_per_token(shape, ctx_len):
    """Algorithmic HBM bytes of one decode step: every weight byte once (tied LM head
    read once as the LM head; the embedding row is one row) + K/V of ctx_len rows."""
    H, I, L, V = shape.hidden, shape.inter, shape.layers, shape.vocab
    qkv = (shape.q_dim + 2 * shape.kv_dim) * (H + 1)     # weights + bias
    per_layer = (qkv + shape.q_dim * H + 2 * I * H + I * H + 2 * H) * 2
    kv = 2 * ctx_len * shape.kv_dim * 2 * L
    return L * per_layer + V * H * 2 + H * 2 + H * 2 + kv

ROOFLINE_KERNEL = "efm_decode_norm_gate_up_swiglu (gemv_kernel<1,1,PRO_ADD_NORM,EPI_SWIGLU>)"
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gate_up_swiglu_c2_hbm_traffic.md")


def gate_up_bytes(shape):
    """Algorithmic bytes of one fused norm + gate/up + SwiGLU launch: the [2I, H] bf16
    weight, the activation, residual in/out and norm weight (H each), the [I] output."""
    H, I = shape.hidden, shape.inter
    return 2 * I * H * 2 + (3 * H + H + I) * 2


def measured_traffic():
    """HBM bytes per launch of the roofline kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def roofline_kernel(torch, C, shape, weights, dev, graph=True, reps=20):
    """Times the fused norm + gate/up GEMV + SwiGLU kernel over all layers' weights
    (1.5 GB, so no launch finds its weight in the 256 MB Infinity Cache). With graph=True
    the reps x layers launches are captured in one HIP graph and replayed between two
    HIP events on the replay stream, so host launch cost stays out of the average; the
    figure is kernel duration plus the graph's inter-node gap."""
    H, I = shape.hidden, shape.inter
    gu = [torch.cat([weights[f"model.layers.{l}.mlp.up_proj.weight"], weights[f"model.layers.{l}.mlp.gate_proj.weight"]])
          for l in range(shape.layers)]
    a = torch.randn(1, H, device=dev).to(torch.bfloat16)
    r_in = torch.randn(1, H, device=dev).to(torch.bfloat16)
    r_out = torch.empty_like(r_in)
    nw = torch.ones(H, device=dev, dtype=torch.bfloat16)
    mid = torch.empty(1, I, device=dev, dtype=torch.bfloat16)

    def launch(l, sh):
        C.call("efm_decode_norm_gate_up_swiglu", H, I, shape.eps, a.data_ptr(), r_in.data_ptr(), r_out.data_ptr(),
               nw.data_ptr(), gu[l].data_ptr(), mid.data_ptr(), sh)

    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    if not graph:
        with torch.cuda.stream(stream):
            for _ in range(reps):
                for l in range(shape.layers):
                    launch(l, stream.cuda_stream)
        stream.synchronize()
        return None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
        for _ in range(reps):
            for l in range(shape.layers):
                launch(l, stream.cuda_stream)
    with torch.cuda.stream(stream):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * shape.layers)
    nbytes = gate_up_bytes(shape)
    gbs = nbytes / (us * 1e-6) / 1e9
    del g, gu
    return {"kernel": ROOFLINE_KERNEL, "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "avg_launch_us": round(us, 3), "bytes_per_launch": nbytes,
            "timing": f"HIP events around one replay of a graph of {reps}x{shape.layers} launches"}


def kernel_only(torch, C, S, shape, seed):
    """Counter-collection workload: a 256 MiB device copy (calibration: 262144 KiB read,
    262144 KiB written) then 2 x layers direct launches of the roofline kernel."""
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x = torch.empty(128 << 20, dtype=torch.bfloat16, device=dev).uniform_()
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    weights = S.synthetic_weights_gpu(shape, seed=seed)
    roofline_kernel(torch, C, shape, weights, dev, graph=False, reps=2)
    torch.cuda.synchronize()
    print(json.dumps({"kernel_only": ROOFLINE_KERNEL, "launches": 2 * shape.layers,
                      "bytes_per_launch": gate_up_bytes(shape), "copy_calibration_bytes": 256 << 20}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--gen", type=int, default=256)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only the copy calibration and the roofline kernel (for rocprofv3 --pmc passes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the single-request decode path of this build runs on one MI355X; "
              "multi-GPU sharding is design-only (see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import edge_fm
    import efm_capi as C
    import efm_setup as S

    shape = S.QWEN25_1P5B
    if args.kernel_only:
        kernel_only(torch, C, S, shape, args.seed)
        return
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    weights = S.synthetic_weights_gpu(shape, seed=args.seed)
    S.register_weights(weights)
    g = torch.Generator().manual_seed(args.seed)
    prompt = torch.randint(0, shape.vocab, (args.prompt,), generator=g).tolist()

    tmp = tempfile.mkdtemp(prefix="efm_bench_")
    mdir = S.write_model_dir(os.path.join(tmp, "model"), shape)
    ecfg = S.write_engine_config(os.path.join(tmp, "engine.json"), mdir, max_tokens=args.prompt + args.gen,
                                 max_new_tokens=args.gen, use_graph=True)
    eng = edge_fm.EdgeFM(ecfg)
    req = edge_fm.Request(0, prompt)
    req.set_ignore_stop_tokens(True)

    for _ in range(args.warmup):
        eng.generate(req)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    mets, toks = [], None
    for _ in range(args.steps):
        toks = eng.generate(req).token_ids()
        mets.append(eng.last_generate_metrics())
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    dec_steps = sum(m["decode_steps"] for m in mets)
    dec_ms = sum(m["decode_ms"] for m in mets)
    pf_ms = sum(m["prefill_ms"] for m in mets)
    decode_tps = dec_steps * 1000.0 / dec_ms
    prefill_tps = args.prompt * len(mets) * 1000.0 / pf_ms
    ms_per_token = dec_ms / dec_steps
    mean_ctx = args.prompt + (args.gen + 1) / 2.0
    bytes_tok = decode_bytes_per_token(shape, mean_ctx)
    loop_gbs = bytes_tok / (ms_per_token * 1e-3) / 1e9

    kern = roofline_kernel(torch, C, shape, weights, dev, graph=True)

    # ---- CPU baseline: the oracle on this host, bounded sample
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import efm_oracle as O

        ocfg = O.QwenConfig(hidden=shape.hidden, layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                            head_dim=shape.head_dim, inter=shape.inter, vocab=shape.vocab)
        wcpu = {k: v.cpu() for k, v in weights.items()}
        orc = O.Qwen2Oracle(ocfg, O.fuse_weights(ocfg, wcpu), max_tokens=16 + 48 + 8, cache_f32=True)
        del wcpu
        st = orc.new_state()
        orc.forward(st, torch.tensor(prompt[:16], dtype=torch.int32))
        n_dec = 48
        c0 = time.perf_counter()
        for i in range(n_dec):
            orc.forward(st, torch.tensor([toks[i]], dtype=torch.int32))
        c_s = time.perf_counter() - c0
        cpu = {"value": round(n_dec / c_s, 3), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"CPU oracle (PyTorch fp32 math on bf16 values), same 1.5B-shaped weights, 16-token "
                         f"prefill then {n_dec} decode steps at context 17-{16 + n_dec}; decode tokens/s"}

    line = {
        "metric": "bs=1 decode tokens/s (Qwen2.5-1.5B shape, greedy, 512-token prompt + 256 generated)",
        "value": round(decode_tps, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1000.0 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) bf16 weights, uniform random prompt ids)",
        "config": {"workload": "C2: Qwen2.5-1.5B-shaped decoder, bs=1 greedy, prompt 512, 256 generated tokens",
                   "layers": shape.layers, "hidden": shape.hidden, "heads": f"{shape.heads}/{shape.kv_heads}",
                   "head_dim": shape.head_dim, "intermediate": shape.inter, "vocab": shape.vocab,
                   "prompt": args.prompt, "generated": args.gen, "hip_graph": True},
        "prefill_tokens_per_s": round(prefill_tps, 1),
        "decode_ms_per_token": round(ms_per_token, 4),
        "decode_loop": {"bytes_per_token": int(bytes_tok), "achieved_GBs": round(loop_gbs, 1),
                        "frac_of_hbm_peak": round(loop_gbs / HBM_PEAK_GBS, 4)},
        "roofline": kern,
        "cpu_baseline": cpu,
        "tokens_head": toks[:8],
    }
    print(json.dumps(line))
    del eng


if __name__ == "__main__":
    main()
