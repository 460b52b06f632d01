"""INT4-KV decode-attention benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Workload (one step = one launch of the split-K decode kernel over one batch):
single-layer decode attention, batch 1, 32 query heads / 8 kv heads (GQA),
head_dim 128, context 32768 = 64 fp16 sink tokens + 28608 INT4 tokens (16-token
blocks) + 4096 fp16 recent tokens; q ~ N(0,1)/sqrt(128) fp16; K, V ~ N(0,1) fp16
with K channels 7/31/64/100 scaled x8; seeded, synthetic.  Eight copies of the
KV are rotated (8 x 48.6 MB > the 256 MB Infinity Cache) so reads come from HBM.
Launches are replayed from a HIP graph.

Prints one JSON line: value = algorithmic bytes per step x steps / elapsed (GB/s),
a roofline object for the decode kernel (achieved GB/s vs the 8 TB/s HBM peak,
kernel time from HIP events on the launch stream) and a cpu_baseline object (the
oracle's dequantize-then-attend restatement timed on the host cores).
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hetero-kvcache-optimizer_amd"))

METRIC = "INT4-KV decode-attn GB/s (% HBM peak) at 32K ctx; tok/s at 128K w/ offload"
HBM_PEAK_GBS = 8000.0
B, HQ, HKV, D = 1, 32, 8, 128
SINK, MID, RECENT = 64, 28608, 4096
CTX = SINK + MID + RECENT
OUTLIERS = [7, 31, 64, 100]
# Algorithmic bytes per step: packed INT4 codes + per-token fp32 scale / u8 zp for K and V,
# the fp16 sink + recent K and V, the fp16 query and the fp16 output.
BYTES_CODES = 2 * HKV * MID * (D // 2)
BYTES_META = 2 * HKV * MID * 5
BYTES_F16 = 2 * HKV * (SINK + RECENT) * D * 2
BYTES_QO = 2 * B * HQ * D * 2
STEP_BYTES = BYTES_CODES + BYTES_META + BYTES_F16 + BYTES_QO  # 48,638,976
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_attn_c2_traffic.txt")


def make_inputs(torch, seed=2):
    g = torch.Generator().manual_seed(seed)
    K = torch.randn((B, HKV, CTX, D), generator=g)
    K[..., OUTLIERS] *= 8
    V = torch.randn((B, HKV, CTX, D), generator=g)
    q = torch.randn((B, HQ, D), generator=g) / math.sqrt(D)
    return q.half(), K.half(), V.half()


def build_copy(torch, ops, q, K, V, dev):
    sink = ops.F16Zone(B, HKV, SINK, dev)
    sink.write(K[:, :, :SINK].to(dev), V[:, :, :SINK].to(dev), [0])
    rec = ops.F16Zone(B, HKV, RECENT, dev)
    rec.write(K[:, :, SINK + MID:].to(dev), V[:, :, SINK + MID:].to(dev), [0])
    nb = (MID + 15) // 16
    pool = ops.Int4Pool(nb, HKV, dev)
    bt = torch.arange(nb, dtype=torch.int32, device=dev)[None]
    ops.pack_tokens(pool, K[:, :, SINK:SINK + MID].to(dev), V[:, :, SINK:SINK + MID].to(dev),
                    torch.zeros(1, dtype=torch.int32, device=dev), bt)
    pool.check_errors()
    return dict(zones=[(sink, None, SINK), (rec, None, RECENT)], pool=pool, bt=bt)


def read_traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (committed summary), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return float(ln.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(q, K, V, budget_s=10.0):
    """The oracle's dequantize-then-attend (Path C semantics) on the host cores."""
    import numpy as np
    from oracle import attention as oa
    from oracle import compressor as oc
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    except Exception:
        threads = 1
    kn, vn = K[0].numpy(), V[0].numpy()
    kc, ks, kz = oc.compress(kn[:, SINK:SINK + MID], 128)
    vc, vs, vz = oc.compress(vn[:, SINK:SINK + MID], 128)
    qn = q[0].double().numpy()[:, None]
    hbm_k = np.concatenate([kn[:, :SINK], kn[:, SINK + MID:]], axis=1).astype(np.float64)
    hbm_v = np.concatenate([vn[:, :SINK], vn[:, SINK + MID:]], axis=1).astype(np.float64)

    def step():
        kd = oa.dequant_rows(kc, ks.reshape(HKV, MID), kz.reshape(HKV, MID))
        vd = oa.dequant_rows(vc, vs.reshape(HKV, MID), vz.reshape(HKV, MID))
        return oa.attend(qn, np.concatenate([kd, hbm_k], 1), np.concatenate([vd, hbm_v], 1))

    out = step()  # warmup
    n, t0 = 0, time.perf_counter()
    while True:
        out = step()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 50:
            break
    return out, dict(value=STEP_BYTES * n / el / 1e9, unit="GB/s", cores=threads, kind="port",
                     sample="%d full C2 decode steps (dequant INT4 -> fp16 -> float64 attention) in %.1f s"
                            % (n, el))


P_SQ, P_SINK, P_MID, P_RECENT = 2048, 64, 131072, 4096
# 4*Hq*D per (query, visible key): history fully visible, the chunk causally
P_FLOPS = 4 * HQ * D * P_SQ * (P_SINK + P_MID + P_RECENT) + 4 * HQ * D * (P_SQ * (P_SQ + 1) // 2)
MFMA_PEAK_TFLOPS = 2500.0


def bench_prefill(torch, ops, args):
    """One step = one hkv_prefill_attn launch: 2048 fp16 queries (32 q / 8 kv heads) against
    64 fp16 sink + 131072 INT4 + 4096 fp16 recent tokens plus the chunk itself (causal)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(4)
    hist = P_SINK + P_MID + P_RECENT
    K = torch.randn((1, HKV, hist, D), generator=g, device=dev)
    K[..., OUTLIERS] *= 8
    K = K.half()
    V = torch.randn((1, HKV, hist, D), generator=g, device=dev).half()
    CK = torch.randn((1, HKV, P_SQ, D), generator=g, device=dev).half()
    CV = torch.randn((1, HKV, P_SQ, D), generator=g, device=dev).half()
    q = (torch.randn((1, HQ, P_SQ, D), generator=g, device=dev) / math.sqrt(D)).half()
    sink = ops.F16Zone(1, HKV, P_SINK, dev)
    sink.write(K[:, :, :P_SINK], V[:, :, :P_SINK], [0])
    rec = ops.F16Zone(1, HKV, P_RECENT, dev)
    rec.write(K[:, :, P_SINK + P_MID:], V[:, :, P_SINK + P_MID:], [0])
    nb = P_MID // 16
    pool = ops.Int4Pool(nb, HKV, dev)
    bt = torch.arange(nb, dtype=torch.int32, device=dev)[None]
    ops.pack_tokens(pool, K[:, :, P_SINK:P_SINK + P_MID], V[:, :, P_SINK:P_SINK + P_MID],
                    torch.zeros(1, dtype=torch.int32, device=dev), bt)
    del K, V
    out = torch.empty((1, HQ, P_SQ, D), dtype=torch.float16, device=dev)
    zones = [(sink, None, P_SINK), (rec, None, P_RECENT)]

    def launch():
        ops.prefill_attention(q, zones=zones, pool=pool, block_table=bt, int4_max_len=P_MID,
                              chunk_k=CK, chunk_v=CV, out=out)

    for _ in range(max(args.warmup, 1)):
        launch()
    torch.cuda.synchronize()
    pool.check_errors()
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(args.steps):
        launch()
    ev1.record(stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    tflops = P_FLOPS / (ms * 1e-3) / 1e12
    line = {
        "metric": "INT4-KV chunked-prefill attention TFLOP/s (MFMA roofline fraction)",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (seeded N(0,1) K/V, x8 K outlier channels)",
        "config": {"workload": "chunked prefill: 2048 fp16 queries, 32 q / 8 kv heads, head_dim 128, over "
                               "64 fp16 sink + 131072 INT4 + 4096 fp16 recent + causal chunk",
                   "flops_per_step": P_FLOPS},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_PEAK_TFLOPS, 4), "traffic": None},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--workload", choices=["decode", "prefill"], default="decode",
                    help="decode: the headline single-layer decode (default); prefill: the chunked-prefill "
                         "kernel on a 2048-token chunk over 64 + 131072 INT4 + 4096 tokens (MFMA bound)")
    ap.add_argument("--copy-calibration", type=float, default=0.0,
                    help="run only torch's device copy of this many MB (20 launches) so that rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE can be scaled against a known byte count")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the decode path shards by kv head or "
              "sequence with no exchange; see DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration > 0:
        dev = torch.device("cuda:0")
        n = int(args.copy_calibration * 1e6) // 4
        src = torch.ones(n, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read_per_launch": n * 4,
                          "copy_calibration_bytes_written_per_launch": n * 4, "launches": 20}), flush=True)
        return

    from heterokv import ops

    if args.workload == "prefill":
        return bench_prefill(torch, ops, args)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, K, V = make_inputs(torch)
    R = args.copies
    copies = [build_copy(torch, ops, q, K, V, dev) for _ in range(R)]
    q_dev = q.to(dev)
    out = torch.empty((B, HQ, D), dtype=torch.float16, device=dev)
    ws = ops.DecodeWorkspace(dev)

    def launch(i):
        c = copies[i % R]
        ops.decode_attention(q_dev, zones=c["zones"], pool=c["pool"], block_table=c["bt"],
                             int4_max_len=MID, workspace=ws, out=out)

    for i in range(max(R, 8)):
        launch(i)
    torch.cuda.synchronize()

    stream = torch.cuda.Stream(device=dev)
    K_steps, W = args.steps, args.warmup
    graphs = {}
    if not args.no_graph:
        def capture(n):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(n):
                    launch(i)
            return g
        graphs["full"] = capture(R)
        if K_steps % R:
            graphs["rem"] = capture(K_steps % R)
        if W % R:
            graphs["wrem"] = capture(W % R)

    def run(n, rem_key):
        if args.no_graph:
            with torch.cuda.stream(stream):
                for i in range(n):
                    launch(i)
            return
        for _ in range(n // R):
            graphs["full"].replay()
        if n % R:
            graphs[rem_key].replay()

    with torch.cuda.stream(stream):
        run(W, "wrem")
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
        run(K_steps, "rem")
        ev1.record(stream)
    ev1.synchronize()
    torch.cuda.synchronize()
    ms_total = ev0.elapsed_time(ev1)
    ms_step = ms_total / K_steps
    gbs = STEP_BYTES * K_steps / (ms_total * 1e-3) / 1e9
    if ws.error_flag():
        raise RuntimeError("decode kernel reported an out-of-range block id")

    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np
        ref, cpu = cpu_baseline(q, K, V, args.cpu_budget)
        launch(0)
        torch.cuda.synchronize()
        err = float(np.abs(out[0].float().cpu().numpy() - ref[:, 0]).max())
        if not err <= 2e-3:
            raise RuntimeError("GPU output differs from the oracle by %.3e" % err)

    traffic = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": W,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) K/V with x8 K outlier channels; INT4 middle packed by the "
                "build's quantizer)",
        "config": {"workload": "single-layer INT4-KV decode attention, batch 1, 32 q / 8 kv heads, "
                               "head_dim 128, ctx 32768 = 64 fp16 sink + 28608 INT4 + 4096 fp16 recent",
                   "batch": B, "context": CTX, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "int4_tokens": MID, "fp16_tokens": SINK + RECENT, "kv_copies_rotated": R,
                   "launch": "eager" if args.no_graph else "hip graph replay",
                   "bytes_per_step": STEP_BYTES},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "cpu_baseline": ({k: (round(v, 4) if isinstance(v, float) else v) for k, v in cpu.items()}
                         if cpu else None),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
