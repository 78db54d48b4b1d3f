"""Benchmark of the MI355X DSA-layer hot path: one JSON line on stdout.

Workload (N = 1, the default ``--workload layer``): BASELINE.json configs[4], one GPU's
TP=4 share of a DeepSeek-V3.2 DSA decoder layer at 8 decode rows, each row its own
request at position 32767 (context 32768): the front (RMSNorm, q_a | kv_a, q_b, RoPE,
W_UK, the KV and FP4 index-key cache writes, the FP4 index query), the attention phase
(FP4 indexer scores, exact top-2048, sparse MLA), the output block (W_UV, o_proj,
residual) and the FP8 MoE (RMSNorm, router, top-8 + shared experts, residual), as ONE
persistent launch a layer (``mono_layer_launch``). A step is one layer over one batch;
``--layers`` independently seeded layers (about 3 GB each, 0.5 GB of it touched a step,
so the 256 MB MALL cannot serve them) are rotated. Inputs are resident in HBM before the
timed region; the timed region replays a HIP graph of every layer's launch, is bracketed
by ``torch.cuda.synchronize()`` and is measured with HIP events on the replay stream.
``value`` is the average µs per layer.

``roofline``: the layer kernel's (the step's only kernel) algorithmic bytes per launch --
the front's, output block's and router's weights, every distinct expert the batch routed
to (shared included) x 11,012,736 B, the KV rows gathered and index keys scanned, the
rows in and out -- over its average launch time, against 8 TB/s. ``config`` also gives
each phase's end inside the launch (timeline stamps) and each phase's time and achieved
bandwidth as a launch of its own (the four-launch chain). ``cpu_baseline``: the CPU oracle chain
(``oracle/front.py``, ``oracle/attn.py``, ``oracle/dense.py``, ``oracle/moe.py``) for the
whole layer at all rows on this host's cores (the box's thread share), one warm-up then
the median of five runs, with the core count and CPU model.

Other workloads (``--workload``): moe_fp8 (configs[1] alone), moe_mxfp4,
attn, post (the output block alone).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "µs per decoder layer at 8 rows; MoE/attn achieved HBM TB/s vs 8 TB/s peak"
HBM_PEAK_GBS = 8000.0
EXPERT_BYTES = 7_340_032 + 1_792 + 3_670_016 + 896  # w13 + s13 + w2 + s2 of one expert
ROUTER_BYTES = 3_670_016
# MXFP4 expert of config 4: w13 768 x 1536 B + 768 x 96 scales, w2 3072 x 192 B + 3072 x 12
MX_EXPERT_BYTES = 1_179_648 + 73_728 + 589_824 + 36_864
# MXFP4 expert at the layer's geometry: w13 1024 x 3584 B + 1024 x 224, w2 7168 x 256 + 7168 x 16
MX_LAYER_EXPERT_BYTES = 3_670_016 + 229_376 + 1_835_008 + 114_688


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=40)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="layer",
                   choices=("layer", "moe_fp8", "moe_mxfp4", "attn", "post"),
                   help="layer: BASELINE configs[4], the full decoder layer (the metric); "
                        "moe_fp8: configs[1], the FP8 MoE phase alone; "
                        "moe_mxfp4: configs[3], the MXFP4 A16W4 expert block; "
                        "attn: configs[2], FP4 indexer + top-2048 + sparse MLA; "
                        "post: W_UV + o_proj + residual")
    p.add_argument("--ctx", type=int, default=32768, help="attn: keys each row sees")
    p.add_argument("--rows", type=int, default=8)
    p.add_argument("--layers", type=int, default=4)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--layout", default="aiter16", choices=("aiter16", "rowmajor"),
                   help="on-HBM layout of the expert weights (SGLang's gfx950 MoE load "
                        "leaves them in AITER's (16, 16) shuffle)")
    p.add_argument("--index-format", default="fp4", choices=("fp4", "dsa"),
                   help="layer / attn: the index keys in the FP4 index plane (BASELINE "
                        "configs[2], the default) or in SGLang's DSA pages (E4M3 + per-token "
                        "scales, 16x16 tiles; bf16 index query)")
    p.add_argument("--experts", default="fp8", choices=("fp8", "mxfp4"),
                   help="layer: the MoE's experts, FP8 W8A8 (BASELINE configs[4]) or MXFP4 "
                        "A16W4 (E2M1 + E8M0 per 32) in the same one launch")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a 1 GiB device-to-device copy 5 times (the reference "
                        "point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    return p.parse_args()


def copy_calibration():
    import torch

    n = 1 << 30
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "launches": 5}), flush=True)


def traffic_from_profiles(name: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    f = ROOT / "profiles" / f"{name}_traffic.json"
    if f.exists():
        try:
            return json.loads(f.read_text()).get("bytes_per_launch")
        except (OSError, ValueError):
            return None
    return None


def cpu_threads() -> int:
    """Host threads for the CPU leg: the box's share (OMP_NUM_THREADS), else every core."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def cpu_model() -> str:
    """The host CPU's model name (lscpu's, from /proc/cpuinfo)."""
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.lower().startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_timed(fn, runs: int = 5):
    """One warm-up call, then the median of ``runs`` timed calls (perf_counter), as the
    CPU-baseline plan asks. Returns (median s, every run's s)."""
    import statistics

    import torch

    torch.set_num_threads(cpu_threads())
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


def cpu_record(value_us: float, unit: str, sample: str, times) -> dict:
    import torch

    return {"value": round(value_us, 1), "unit": unit, "cores": torch.get_num_threads(),
            "kind": "port", "sample": sample, "cpu_count": os.cpu_count(),
            "cpu_model": cpu_model(), "runs_s": [round(t, 3) for t in times]}


def cpu_baseline_mxfp4(x_cpu, logits_cpu, w, ids, rows):
    """The oracle's MXFP4 block on the host, one launch worth (bounded sample)."""
    import numpy as np
    import torch

    from oracle import moe as omoe
    from sgl_amd_mono_amd.dsv32 import synthetic

    experts = {int(e): synthetic.rowmajor_mxfp4_expert(w, int(e)) for e in np.unique(ids)}
    parts = [{e: v[k] for e, v in experts.items()} for k in range(4)]
    med, times = cpu_timed(lambda: omoe.moe_mxfp4(x_cpu, logits_cpu, w.bias.cpu(), *parts,
                                                  residual=x_cpu))
    return cpu_record(med * 1e6, f"µs per MXFP4 MoE block ({rows} rows)",
                      f"the whole block: {rows} rows over their {len(experts)} routed experts "
                      f"(oracle/moe.py, f64 GEMVs on dequantised E2M1), one warm-up then the "
                      f"median of {len(times)} runs", times)


def cpu_baseline(a_cpu, w, ids, rows):
    """The oracle's MoE block on the host, one launch worth (bounded sample)."""
    import numpy as np
    import torch

    from oracle import moe as omoe

    from sgl_amd_mono_amd.dsv32 import synthetic

    experts = {int(e): synthetic.rowmajor_expert(w, int(e)) for e in np.unique(ids)}
    args = (a_cpu, w.g_post.cpu(), w.w_r.cpu(), w.bias.cpu(), None, None, None, None)
    med, times = cpu_timed(lambda: omoe.moe_fp8(*args, experts=experts))
    return cpu_record(med * 1e6, f"µs per MoE block ({rows} rows)",
                      f"the whole block: {rows} rows over their {len(experts)} routed experts "
                      f"(oracle/moe.py, f64 GEMVs on dequantised E4M3), one warm-up then the "
                      f"median of {len(times)} runs", times)


def time_graph(launch, L: int, steps: int, warmup: int):
    """Average µs of one launch: a HIP graph holds a launch on each of the L layers in
    turn (as the reference's timing harness replays a captured step of launches,
    test/kernels/glm53/time_layers.py:38-76) and the timed region replays it, so the
    host issues nothing per launch. Eager warm-up first, then graph warm-up replays.
    HIP events bracket the replays on the replay stream. Returns (us, wall_s, steps)."""
    import torch

    for s in range(warmup):
        launch(s % L)
    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        for i in range(L):  # warm-up on the capture stream
            launch(i)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=cs):
        for i in range(L):
            launch(i)
    reps = max(1, steps // L)
    for _ in range(max(1, warmup // L)):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(reps):
        graph.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) * 1e3 / (reps * L), wall, reps * L


def bench_moe_fp8(args):
    import numpy as np
    import torch

    from sgl_amd_mono_amd.dsv32 import synthetic
    from sgl_amd_mono_amd.dsv32.config import DSV32
    from sgl_amd_mono_amd.dsv32.moe import MoeFp8Op, MoeRouting

    dev = torch.device("cuda:0")
    rows, L = args.rows, args.layers
    print(f"bench: generating {L} layers of FP8 experts", file=sys.stderr, flush=True)
    weights = [synthetic.moe_fp8_weights(dev, seed=100 + i, layout=args.layout) for i in range(L)]
    ops = [MoeFp8Op(w, dev, max_rows=rows) for w in weights]
    inputs = [synthetic.rows_bf16(rows, DSV32.hidden, dev, seed=200 + i) for i in range(L)]
    outs = [torch.empty(rows, DSV32.hidden, dtype=torch.bfloat16, device=dev) for _ in range(L)]

    # routing of each (layer, batch): the distinct experts a launch streams
    distinct = []
    ids0 = None
    for i in range(L):
        rt = MoeRouting(torch.empty(rows, DSV32.experts, device=dev),
                        torch.empty(rows, 9, dtype=torch.int32, device=dev),
                        torch.empty(rows, 9, device=dev))
        ops[i].launch(inputs[i], routing=rt, out=outs[i])
        ops[i].rt.check()
        ids = rt.ids.cpu().numpy()
        distinct.append(len(np.unique(ids)))
        if i == 0:
            ids0 = ids
    act_bytes = rows * DSV32.hidden * 2 * 2
    bytes_per = [d * EXPERT_BYTES + ROUTER_BYTES + act_bytes for d in distinct]

    us, wall, steps = time_graph(lambda i: ops[i].launch(inputs[i], out=outs[i]), L,
                                 args.steps, args.warmup)
    for op in ops:
        op.rt.check()
    print(f"bench: {steps} launches, {us:.1f} us each (wall {wall * 1e3 / steps:.1f} "
          f"ms/step), distinct experts {distinct}", file=sys.stderr, flush=True)
    cpu = None if args.no_cpu else cpu_baseline(inputs[0].cpu(), weights[0], ids0, rows)
    config = {
        "workload": "BASELINE configs[1]: FP8 routed MoE, one GPU's TP=4 share, one "
                    "persistent launch (post-norm, router, top-8 + shared, W8A8 SwiGLU, "
                    "down, residual)",
        "rows": rows, "hidden": DSV32.hidden, "experts": DSV32.experts + 1,
        "inter": DSV32.inter, "layers_rotated": L, "weight_layout": args.layout,
        "distinct_experts": distinct,
    }
    return us, steps, sum(bytes_per) / L, "fp8", config, "moe_fp8_r8", cpu


def bench_moe_mxfp4(args):
    import numpy as np
    import torch

    from sgl_amd_mono_amd.dsv32 import synthetic
    from sgl_amd_mono_amd.dsv32.config import MXFP4_MOE as C
    from sgl_amd_mono_amd.dsv32.moe import MoeMxfp4Op, MoeRouting

    dev = torch.device("cuda:0")
    rows, L = args.rows, args.layers
    print(f"bench: generating {L} layers of MXFP4 experts", file=sys.stderr, flush=True)
    weights = [synthetic.mxfp4_moe_weights(dev, seed=100 + i, layout=args.layout)
               for i in range(L)]
    ops = [MoeMxfp4Op(w, dev, max_rows=rows) for w in weights]
    xs = [synthetic.rows_bf16(rows, C.hidden, dev, seed=300 + i) for i in range(L)]
    logits = [synthetic.logits_f32(rows, C.experts, dev, seed=300 + i) for i in range(L)]
    outs = [torch.empty(rows, C.hidden, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    distinct, ids0 = [], None
    for i in range(L):
        rt = MoeRouting(torch.empty(rows, C.experts, device=dev),
                        torch.empty(rows, 9, dtype=torch.int32, device=dev),
                        torch.empty(rows, 9, device=dev))
        ops[i].launch(xs[i], logits[i], res=xs[i], routing=rt, out=outs[i])
        ops[i].rt.check()
        ids = rt.ids.cpu().numpy()
        distinct.append(len(np.unique(ids)))
        if i == 0:
            ids0 = ids
    # rows in, residual in, out; logits
    act_bytes = rows * C.hidden * 2 * 3 + rows * C.experts * 4
    bytes_per = [d * MX_EXPERT_BYTES + act_bytes for d in distinct]
    us, wall, steps = time_graph(
        lambda i: ops[i].launch(xs[i], logits[i], res=xs[i], out=outs[i]), L, args.steps,
        args.warmup)
    for op in ops:
        op.rt.check()
    print(f"bench: {steps} launches, {us:.1f} us each (wall {wall * 1e3 / steps:.1f} "
          f"ms/step), distinct experts {distinct}", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_mxfp4(xs[0].cpu(), logits[0].cpu(), weights[0], ids0, rows)
    config = {
        "workload": "BASELINE configs[3]: MXFP4 (A16W4) routed MoE, one GPU's TP=4 share, "
                    "one persistent launch (given logits, sigmoid + bias top-8 + shared, "
                    "E2M1/E8M0 SwiGLU with bf16 mid, down, residual)",
        "rows": rows, "hidden": C.hidden, "experts": C.experts + 1, "inter": C.inter,
        "layers_rotated": L, "weight_layout": args.layout, "distinct_experts": distinct,
    }
    return us, steps, sum(bytes_per) / L, "bf16 x e2m1", config, f"moe_mxfp4_r{rows}", cpu


def cpu_baseline_attn(inp, sm_scale, rows):
    """The oracle's attention chain on the host for every row of the launch."""
    from oracle import attn as A

    plane, psc = inp.plane.cpu().numpy(), inp.plane_scale.cpu().numpy()
    kv = inp.kv.cpu().numpy()
    ksc = None if inp.kv_scale is None else inp.kv_scale.cpu().numpy()
    per_row = [(inp.q[r].cpu(), inp.iq[r].cpu().numpy(), inp.iqs[r].cpu().numpy(),
                inp.iw[r].cpu().numpy(), plane, psc,
                inp.page_table[int(inp.req_ids[r])].cpu().numpy(), kv, ksc,
                int(inp.positions[r]), 2048, sm_scale) for r in range(rows)]
    med, times = cpu_timed(lambda: [A.attention_row(*a) for a in per_row])
    return cpu_record(med * 1e6, f"µs per attention phase ({rows} rows)",
                      f"all {rows} rows (f64 numpy/torch: scores of "
                      f"{int(inp.positions[0]) + 1} keys, exact top-2048, sparse MLA), one "
                      f"warm-up then the median of {len(times)} runs", times)


def bench_attn(args):
    import torch

    from sgl_amd_mono_amd import _lib
    from sgl_amd_mono_amd.dsv32 import synthetic
    from sgl_amd_mono_amd.dsv32.attn import AttnOp

    dev = torch.device("cuda:0")
    rows, L, ctx = args.rows, args.layers, args.ctx
    print(f"bench: generating {L} layers of caches ({rows} rows x {ctx} keys)", file=sys.stderr,
          flush=True)
    dsa = args.index_format == "dsa"
    fmt = _lib.INDEX_FP8_PAGE if dsa else _lib.INDEX_FP4_PLANE
    inps = [synthetic.attention_inputs(rows, ctx, dev, seed=400 + i, index_format=fmt)
            for i in range(L)]
    ops = [AttnOp(dev, max_rows=rows, ctx_max=ctx) for _ in range(L)]
    outs = [torch.empty(rows, 32, 512, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    n = min(ctx, 1 << 30)
    k = min(n, 2048)
    # KV rows gathered (576 E4M3 + a 4-byte scale), index keys scanned (FP4: 64 B + 4
    # scales; DSA: 128 B + a scale), the queries in (absorbed q bf16, index q (+ scales) +
    # weights) and the latent out
    key, iqb = index_bytes(dsa)
    bytes_per = rows * (k * 580 + n * key + 32 * 576 * 2 + iqb + 64 * 4 + 32 * 512 * 2)
    us, wall, steps = time_graph(lambda i: ops[i].launch(inps[i], out=outs[i]), L, args.steps,
                                 args.warmup)
    for op in ops:
        op.rt.check()
    print(f"bench: {steps} launches, {us:.1f} us each (wall {wall * 1e3 / steps:.1f} ms/step)",
          file=sys.stderr, flush=True)
    # the CPU baseline leg restates the FP4 indexer (the headline configuration)
    cpu = None if args.no_cpu or dsa else cpu_baseline_attn(inps[0], ops[0].sm_scale, rows)
    config = {
        "workload": "BASELINE configs[2]: sparse MLA decode, 32 heads, kv_lora 512 + rope 64, "
                    "64-token paged E4M3 KV with per-token scales, FP4 indexer (64 heads x 128, "
                    "E2M1 + E8M0) top-2048, one persistent launch" if not dsa else
                    "configs[2] geometry over SGLang's DSA index pages: sparse MLA decode, 32 "
                    "heads, 64-token paged E4M3 KV, indexer over E4M3 keys with per-token "
                    "power-of-two scales (16x16 tiles) and a bf16 query, top-2048, one "
                    "persistent launch",
        "rows": rows, "context": ctx, "topk": k, "layers_rotated": L,
        "index_format": args.index_format,
    }
    name = f"attn_r{rows}" if not dsa else f"attn_dsa_r{rows}"
    return (us, steps, bytes_per, "fp4 idx / bf16 x e4m3 attn" if not dsa else
            "bf16 x e4m3 idx / bf16 x e4m3 attn", config, name, cpu)


def cpu_baseline_post(o_lat, h, w):
    """The oracle's W_UV + o_proj + residual on the host for the whole launch."""
    import torch

    from oracle import dense as D
    from sgl_amd_mono_amd.dsv32 import synthetic

    ws = synthetic.rowmajor_post(w)
    o_c, h_c = o_lat.cpu(), h.cpu()
    med, times = cpu_timed(lambda: D.attn_out(o_c, h_c, *ws))
    return cpu_record(med * 1e6, f"µs per attention output block ({o_lat.shape[0]} rows)",
                      "the whole launch: f64 dequantisation of W_UV and W_o and the two GEMVs, "
                      f"one warm-up then the median of {len(times)} runs", times)


def bench_post(args):
    import torch

    from sgl_amd_mono_amd.dsv32 import synthetic
    from sgl_amd_mono_amd.dsv32.post import PostOp

    dev = torch.device("cuda:0")
    rows, L = args.rows, args.layers
    print(f"bench: generating {L} layers of W_UV + o_proj", file=sys.stderr, flush=True)
    ws = [synthetic.post_weights(dev, seed=500 + i, layout=args.layout) for i in range(L)]
    ops = [PostOp(w, dev, max_rows=rows) for w in ws]
    g = torch.Generator(device=dev).manual_seed(5)
    o_lat = torch.randn(rows, 32, 512, generator=g, device=dev).to(torch.bfloat16)
    h = torch.randn(rows, 7168, generator=g, device=dev).to(torch.bfloat16)
    outs = [torch.empty(rows, 7168, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    # E4M3 weights + f32 block scales, o_lat in, h in, a out
    bytes_per = (32 * 128 * 512 + 7168 * 4096 + (32 * 4 + 56 * 32) * 4
                 + rows * (32 * 512 * 2 + 7168 * 2 * 2))
    us, wall, steps = time_graph(lambda i: ops[i].launch(o_lat, h, out=outs[i]), L, args.steps,
                                 args.warmup)
    for op in ops:
        op.rt.check()
    print(f"bench: {steps} launches, {us:.1f} us each (wall {wall * 1e3 / steps:.1f} ms/step)",
          file=sys.stderr, flush=True)
    cpu = None if args.no_cpu else cpu_baseline_post(o_lat, h, ws[0])
    config = {
        "workload": "attention output block: W_UV per head (32 x [128, 512]) and o_proj "
                    "([7168, 4096]), E4M3 + f32 128x128 block scales, bf16 activations, "
                    "residual add, one persistent launch",
        "rows": rows, "layout": args.layout, "layers_rotated": L,
    }
    return us, steps, bytes_per, "bf16 x e4m3", config, f"post_r{rows}", cpu


FRONT_W_BYTES = (2112 * 7168 + 17 * 56 * 4 + 128 * 7168 + 56 * 4 + 64 * 7168 * 2
                 + 6144 * 1536 + 48 * 12 * 4 + 8192 * 1536 + 64 * 12 * 4 + 32 * 512 * 128
                 + 32 * 4 * 4 + (7168 + 1536 + 512) * 2 + 128 * 4 * 2)
POST_W_BYTES = 32 * 128 * 512 + 7168 * 4096 + (32 * 4 + 56 * 32) * 4


def index_bytes(dsa: bool):
    """(bytes a cached index key, bytes of a row's index query): the FP4 plane's 64 B + 4
    E8M0 and 64 x 64 B + 256 E8M0, or a DSA page's 128 B + a 4-byte scale and a bf16
    64 x 128 query."""
    return (132, 64 * 128 * 2) if dsa else (68, 64 * 64 + 256)


def phase_bytes(rows, ctx, distinct, dsa=False, mx=False):
    """Algorithmic bytes of each phase of one layer (each needed byte counted once); ``mx``:
    MXFP4 experts."""
    n, k = ctx, min(ctx, 2048)
    key, iq = index_bytes(dsa)
    front = (FRONT_W_BYTES + rows * (7168 * 2 + 580 + key + 32 * 576 * 2 + iq
                                     + 64 * 4 + 64 * 2 * 2))
    attn = rows * (k * 580 + n * key + 32 * 576 * 2 + iq + 64 * 4 + 32 * 512 * 2)
    post = POST_W_BYTES + rows * (32 * 512 * 2 + 7168 * 2 * 2)
    moe = distinct * (MX_LAYER_EXPERT_BYTES if mx else EXPERT_BYTES) + ROUTER_BYTES + rows * 7168 * 2 * 2
    return {"front": front, "attn": attn, "post": post, "moe": moe}


def cpu_baseline_layer(h, w, caches, step, rows):
    """The oracle chain of one layer on the host for all of its rows: the front, each
    row's attention over its keys, the output block and the MoE over the experts the
    rows route to (dequantised on the fly, as the CPU-baseline plan asks)."""
    import numpy as np
    import torch

    from oracle import attn as A
    from oracle import dense as D
    from oracle import front as Fr
    from oracle import moe as M
    from sgl_amd_mono_amd.dsv32 import synthetic

    fw = synthetic.rowmajor_front(w.front)
    pw = synthetic.rowmajor_post(w.post)
    pos = step.positions.cpu().numpy()
    pt = step.page_table.cpu().numpy()
    rid = step.req_ids.cpu().numpy()
    plane, psc = caches.plane.cpu().numpy(), caches.plane_scale.cpu().numpy()
    kv = caches.kv.cpu().numpy()
    ksc = None if caches.kv_scale is None else caches.kv_scale.cpu().numpy()
    hc = h.cpu()
    g_post, w_r, bias = w.moe.g_post.cpu(), w.moe.w_r.cpu(), w.moe.bias.cpu()
    seen = {}

    def layer():
        f = Fr.front(hc, positions=pos, kv_scaled=ksc is not None, **fw)
        iq, iqs = Fr.iq_bytes(f["iq_codes"], f["iq_e8"])
        o = np.stack([A.attention_row(torch.from_numpy(f["q"][r]).float(), iq[r], iqs[r],
                                      f["iw"][r], plane, psc, pt[rid[r]], kv, ksc, int(pos[r]),
                                      2048, (128 + 64) ** -0.5)["o"] for r in range(rows)])
        o_lat = torch.from_numpy(D.bf16(o)).to(torch.bfloat16)
        a = torch.from_numpy(D.attn_out(o_lat, hc, *pw)["a"]).to(torch.bfloat16)
        ids, _ = M.route_topk(M.sigmoid(M.router_logits(M.rmsnorm(a, g_post), w_r)), bias)
        experts = {e: synthetic.rowmajor_expert(w.moe, e)
                   for e in sorted({int(e) for e in ids.ravel()} | {M.SHARED})}
        seen["experts"] = len(experts)
        M.moe_fp8(a, g_post, w_r, bias, None, None, None, None, experts=experts)

    med, times = cpu_timed(layer)
    return cpu_record(med * 1e6, f"µs per decoder layer ({rows} rows)",
                      f"the whole layer for all {rows} rows through the oracle chain (front, "
                      f"FP4 scores of {int(pos[0]) + 1} keys + exact top-2048 + sparse MLA a "
                      f"row, W_UV/o_proj, router + MoE over the {seen['experts']} experts the "
                      f"rows route to, dequantised on the fly), one warm-up then the median of "
                      f"{len(times)} runs", times)


def layer_timeline(op, h, caches, step, grid):
    """In-launch phase ends of one eager launch (µs from the launch's start, median and
    max over CTAs): the front, attention, output block and MoE done, and the exit."""
    import torch

    from sgl_amd_mono_amd import _lib

    tl = torch.zeros(grid, _lib.TL_COLS, dtype=torch.int64, device=h.device)
    op.launch(h, caches, step, timeline=tl)
    op.check()
    t = tl.cpu().numpy().astype("float64")
    t0 = t[:, 0].min()
    out = {}
    for k, name in enumerate(_lib.TL_LAYER_MARKS[1:], start=1):
        v = (t[:, k] - t0) / 100.0  # 100 MHz clock -> µs
        out[name] = {"median_us": round(float(sorted(v)[len(v) // 2]), 2),
                     "max_us": round(float(v.max()), 2)}
    return out


def bench_layer(args):
    import numpy as np
    import torch

    from sgl_amd_mono_amd import _lib
    from sgl_amd_mono_amd.dsv32 import synthetic
    from sgl_amd_mono_amd.dsv32.attn import AttnInputs
    from sgl_amd_mono_amd.dsv32.layer import FusedLayerOp, LayerDebug, LayerOp, layer_runtime

    dev = torch.device("cuda:0")
    rows, ctx = args.rows, args.ctx
    L = args.layers
    print(f"bench: generating {L} decoder layers ({rows} rows x {ctx} keys)", file=sys.stderr,
          flush=True)
    layers = []
    dsa = args.index_format == "dsa"
    mx = args.experts == "mxfp4"
    fmt = _lib.INDEX_FP8_PAGE if dsa else _lib.INDEX_FP4_PLANE
    for i in range(L):
        layers.append(synthetic.layer(rows, ctx, dev, seed=1000 + i, layout=args.layout,
                                      index_format=fmt, experts=args.experts))
        if (i + 1) % 8 == 0:
            torch.cuda.synchronize()
            print(f"bench: {i + 1} layers ({torch.cuda.memory_allocated() / 2**30:.0f} GiB)",
                  file=sys.stderr, flush=True)
    # the one-launch layers share one runtime, as a served model's layers do
    rt = layer_runtime(dev, max_rows=rows)
    fused = [FusedLayerOp(w, dev, max_rows=rows, ctx_max=ctx, rt=rt) for w, _, _, _ in layers]
    outs = [torch.empty(rows, 7168, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    # the experts each layer's batch routes to (an eager launch with the routing out)
    distinct = []
    for i, (op, (w, caches, step, h)) in enumerate(zip(fused, layers)):
        ids = torch.empty(rows, 9, dtype=torch.int32, device=dev)
        op.launch(h, caches, step, out=outs[i], debug=LayerDebug(ids=ids))
        op.check()
        distinct.append(len(np.unique(ids.cpu().numpy())))
    per = [phase_bytes(rows, ctx, d, dsa, mx) for d in distinct]
    avg = {k: sum(p[k] for p in per) / L for k in per[0]}
    total = sum(avg.values())
    us, wall, steps = time_graph(
        lambda i: fused[i].launch(layers[i][3], layers[i][1], layers[i][2], out=outs[i]), L,
        args.steps, args.warmup)
    rt.check()
    print(f"bench: {steps} layers, {us:.1f} us each as one launch (wall "
          f"{wall * 1e3 / steps:.1f} ms/layer), distinct experts {distinct}", file=sys.stderr,
          flush=True)
    inside = layer_timeline(fused[0], layers[0][3], layers[0][1], layers[0][2], rt.grid)
    print(f"bench: in-launch phase ends {inside}", file=sys.stderr, flush=True)
    dtype = ("mxfp4" if mx else "fp8") + (" / e4m3 idx / bf16" if dsa else " / fp4 idx / bf16")
    prof = "layer" + ("_dsa" if dsa else "") + ("_mx" if mx else "")
    if mx:
        # MXFP4 experts run in the one launch only (no four-launch chain to time beside it)
        config = {
            "workload": "BASELINE configs[4]'s decoder layer with MXFP4 experts: one GPU's "
                        "TP=4 share, 8 rows at position 32767 (context 32768), ONE persistent "
                        "launch a layer: the FP8 front, FP4 indexer + exact top-2048 + sparse "
                        "MLA, W_UV + o_proj + residual, then the MoE over MXFP4 (E2M1 + E8M0 "
                        "per 32) A16W4 experts (norm, router, top-8 + shared, residual)",
            "rows": rows, "context": ctx, "layers_rotated": L, "launches_per_layer": 1,
            "weight_layout": args.layout, "index_format": args.index_format,
            "experts": "mxfp4", "distinct_experts": distinct, "in_launch_phase_ends_us": inside,
            "bytes_per_layer": int(total), "moe_bytes_per_layer": int(avg["moe"]),
            "layer_achieved_GBs": round(total / (us * 1e-6) / 1e9, 1),
        }
        return us, steps, total, dtype, config, prof, None, us
    if L > 8:
        # a model step: one graph replay runs all L distinct layers back to back, so the
        # step's time is measured, not scaled from a rotation of a few layers
        config = {
            "workload": f"a decode step through {L} stacked random-init DSA decoder layers "
                        f"(BASELINE configs[4]), one persistent launch a layer, {rows} rows at "
                        f"context {ctx}, every layer's weights and caches distinct in HBM",
            "rows": rows, "context": ctx, "layers": L, "launches_per_layer": 1,
            "weight_layout": args.layout, "index_format": args.index_format,
            "distinct_experts": distinct, "in_launch_phase_ends_us": inside,
            "bytes_per_layer": int(total),
            "layer_achieved_GBs": round(total / (us * 1e-6) / 1e9, 1),
            "us_per_token_step_measured": round(us * L, 1),
        }
        return us, steps, total, dtype, config, prof, None, us
    # each phase as its own launch (the four-launch chain), for the per-phase figures
    chain = [LayerOp(w, dev, max_rows=rows, ctx_max=ctx) for w, _, _, _ in layers]
    fr_out, att_in, olat, a_in = [], [], [], []
    for i, (op, (w, caches, step, h)) in enumerate(zip(chain, layers)):
        f = op.front.launch(h, caches, step.positions, step.slots)
        inp = AttnInputs(q=f.q, iq=f.iq, iqs=f.iqs, iw=f.iw, plane=caches.plane,
                         plane_scale=caches.plane_scale, kv=caches.kv, kv_scale=caches.kv_scale,
                         positions=step.positions, req_ids=step.req_ids, page_table=step.page_table,
                         index_format=caches.index_format)
        o = op.attn.launch(inp).clone()
        a = op.post.launch(o, h).clone()
        op.moe.launch(a, out=outs[i])
        op.check()
        fr_out.append(f)
        att_in.append(inp)
        olat.append(o)
        a_in.append(a)
    chain_us = time_graph(
        lambda i: chain[i].launch(layers[i][3], layers[i][1], layers[i][2], out=outs[i]), L,
        args.steps, args.warmup)[0]
    phase_us = {
        "front": time_graph(lambda i: chain[i].front.launch(layers[i][3], layers[i][1],
                                                            layers[i][2].positions,
                                                            layers[i][2].slots, out=fr_out[i]),
                            L, args.steps, args.warmup)[0],
        "attn": time_graph(lambda i: chain[i].attn.launch(att_in[i], out=olat[i]), L, args.steps,
                           args.warmup)[0],
        "post": time_graph(lambda i: chain[i].post.launch(olat[i], layers[i][3], out=a_in[i]), L,
                           args.steps, args.warmup)[0],
        "moe": time_graph(lambda i: chain[i].moe.launch(a_in[i], out=outs[i]), L, args.steps,
                          args.warmup)[0],
    }
    for op in chain:
        op.check()
    phases = {k: {"us": round(v, 2), "bytes": int(avg[k]),
                  "achieved_GBs": round(avg[k] / (v * 1e-6) / 1e9, 1)} for k, v in phase_us.items()}
    print(f"bench: four launches {chain_us:.1f} us; phases alone {phases}", file=sys.stderr,
          flush=True)
    # the CPU baseline leg restates the FP4 indexer (the headline configuration)
    cpu = None if args.no_cpu or dsa else cpu_baseline_layer(layers[0][3], layers[0][0],
                                                             layers[0][1], layers[0][2], rows)
    config = {
        "workload": "BASELINE configs[4]: full DeepSeek-V3.2 DSA decoder layer, one GPU's TP=4 "
                    "share, 8 rows at position 32767 (context 32768), ONE persistent launch a "
                    "layer: front (RMSNorm, q_a/kv_a, q_b, RoPE, W_UK, KV + FP4 index-key cache "
                    "writes, FP4 index query), FP4 indexer + exact top-2048 + sparse MLA, W_UV + "
                    "o_proj + residual, FP8 MoE (norm, router, top-8 + shared, residual)",
        "rows": rows, "context": ctx, "layers_rotated": L, "launches_per_layer": 1,
        "weight_layout": args.layout, "index_format": args.index_format,
        "distinct_experts": distinct,
        "in_launch_phase_ends_us": inside,
        "four_launch_chain_us": round(chain_us, 2), "phases_as_own_launches": phases,
        "bytes_per_layer": int(total), "layer_achieved_GBs": round(total / (us * 1e-6) / 1e9, 1),
    }
    # the roofline line is the layer kernel's: the only kernel of the step
    if dsa:
        config["workload"] = config["workload"].replace(
            "KV + FP4 index-key cache writes, FP4 index query), FP4 indexer",
            "KV + DSA index-page writes (E4M3, per-token scales), bf16 index query), DSA "
            "indexer")
    return us, steps, total, dtype, config, prof, cpu, us


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every GPU box here has one GPU, and the sharded "
              f"path (TP=4 exchanges) is not built; got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    run = {"moe_fp8": bench_moe_fp8, "moe_mxfp4": bench_moe_mxfp4, "attn": bench_attn,
           "post": bench_post, "layer": bench_layer}[args.workload]
    res = run(args)
    us, steps, avg_bytes, dtype, config, prof, cpu = res[:7]
    kernel_us = res[7] if len(res) > 7 else us  # the dominant kernel's launch time
    achieved = avg_bytes / (kernel_us * 1e-6) / 1e9  # GB/s
    line = {
        "metric": METRIC,
        "value": round(us, 2),
        "unit": "µs",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": config,
        # rows a second through one launch, or (layer) through the 61 layers of the model
        # (the per-layer time x 61; ``--layers 61`` measures such a step whole)
        "rows_per_s": round(args.rows / (us * 1e-6 * (61 if args.workload == "layer" else 1)), 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(prof),
            "algorithmic_bytes": int(avg_bytes),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
