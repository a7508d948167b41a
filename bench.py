"""Decode-step benchmark on one MI355X: int8 (W8A16) linears + paged-attention decode.

Workload: a Llama-3-8B-shaped int8 weight-only decoder
(32 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, intermediate 14336,
vocab 128256), batch 32, one token per row per step, paged fp16 KV with
block_size 16 in a 16384-block pool, contexts ~ U[128, 4096] drawn with seed 0
(config-2-like), block tables from one randperm of the pool. Weights are random
N(0, 0.02) quantized on the device with the build's int8 format; K/V and
embeddings are random. Inputs are resident in HBM before timing starts.

Prints ONE JSON line. ``value`` = decode tokens/s of the whole step (B tokens per
step), timed over ``--steps`` HIP-graph replays of the step after ``--warmup``
eager steps, the capture and 2 untimed replays. ``roofline`` is for the kernel family with the most time per
step: each family's launches of one step (same inputs, same stream) are captured
into their own graph and replayed ``--kernel-steps`` times back-to-back between
two HIP events, which gives its average launch duration without host launch
latency inside the interval (the single lm_head launch is repeated 8 times in its
graph for the same reason). ``cpu_baseline`` times the CPU oracle on a bounded
sample (one decoder layer at the same batch and contexts, plus an lm_head
slice), extrapolated to the full step. ``hbm_copy`` is a timed 1 GiB
device-to-device copy in the same process: the streaming rate this box reaches,
beside the nominal 8 TB/s peak that ``roofline.frac`` divides by.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "llm-serving-runtime_amd"))
sys.path.insert(0, HERE)

HBM_PEAK_GBPS = 8000.0


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=None, help="rows (default 32; 128 for --workload prefix-batch)")
    ap.add_argument("--workload", choices=["decode", "prefix-batch", "linear-sweep", "attention"], default="decode",
                    help="decode: the headline step (default). prefix-batch: 128 rows in 16 groups of 8 sharing "
                         "a 1024-token prefix (aliased blocks), contexts U[1, 8192], 16 rows finish and 16 join "
                         "every 16 steps. linear-sweep: the single int8 linear (4096x4096, M=1) and the "
                         "Llama-3-8B projections at M in {1, 8, 32, 64}. attention: one paged decode call on "
                         "the config-2 inputs (B 32, contexts U[128, 4096], pool 16384 blocks)")
    ap.add_argument("--model", choices=["llama3-8b", "qwen2-0.5b"], default="llama3-8b")
    ap.add_argument("--layers", type=int, default=None, help="override layer count (diagnostics only)")
    ap.add_argument("--ctx-lo", type=int, default=128)
    ap.add_argument("--ctx-hi", type=int, default=4096)
    ap.add_argument("--pool-blocks", type=int, default=16384)
    ap.add_argument("--kernel-steps", type=int, default=5, help="graph replays per kernel family for kernel timing")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=1)
    ap.add_argument("--traffic-probe", type=int, default=0, metavar="REPS",
                    help="instead of the bench: REPS rounds of the step's paged-attention calls (one per layer, "
                         "bench workload) and a 1 GiB copy, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--stream-shared-kv", action="store_true",
                    help="prefix-batch: read the aliased K/V with streaming loads (no MX_PA_SHARED_BLOCKS), "
                         "for comparison")
    args = ap.parse_args()
    if args.batch is None:
        args.batch = 128 if args.workload == "prefix-batch" else 32
    return args


def cpu_info() -> dict:
    info = {"cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    info["model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return info


def cpu_baseline(shape, batch: int, lens, layers_total: int) -> dict:
    """Time the CPU oracle on one decoder layer (4 dequantized fp32 linears + fp32 paged
    attention over the same contexts) and an lm_head slice; extrapolate to the step."""
    import numpy as np
    import torch

    from oracle import int8_quant, paged_attention

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rng = np.random.default_rng(0)
    s = shape
    mats = {
        "qkv": (s.qkv_out, s.hidden),
        "o": (s.hidden, s.heads * s.head_dim),
        "gate_up": (2 * s.intermediate, s.hidden),
        "down": (s.hidden, s.intermediate),
    }
    weights = {}
    for name, (n, k) in mats.items():
        q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        sc = (np.abs(rng.standard_normal(n)) * 1e-3 + 1e-4).astype(np.float16)
        weights[name] = torch.from_numpy(int8_quant.dequantize(q, sc))
    vocab_slice = 16384
    lm_q = rng.integers(-127, 128, size=(vocab_slice, s.hidden), dtype=np.int8)
    lm_w = torch.from_numpy(int8_quant.dequantize(lm_q, np.full(vocab_slice, 1e-3, np.float16)))
    bs = 16
    lens = [int(x) for x in lens]
    nblk = [math.ceil(x / bs) for x in lens]
    tables = torch.zeros(batch, max(nblk), dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        tables[b, :n] = torch.arange(used, used + n, dtype=torch.int32)
        used += n
    g = torch.Generator().manual_seed(1)
    k_layer = torch.randn(used, s.kv_heads, bs, s.head_dim, generator=g).to(torch.float16)
    v_layer = torch.randn(used, s.kv_heads, bs, s.head_dim, generator=g).to(torch.float16)
    x = torch.randn(batch, s.hidden, generator=g)
    q = torch.randn(batch, s.heads, 1, s.head_dim, generator=g).to(torch.float16)

    def one_layer():
        y = x @ weights["qkv"].T
        attn = paged_attention.decode_rows_fp32(q, k_layer, v_layer, tables, lens, s.head_dim**-0.5, s.group)
        y = attn.reshape(batch, -1) @ weights["o"].T
        gu = x @ weights["gate_up"].T
        a = torch.nn.functional.silu(gu[:, :s.intermediate]) * gu[:, s.intermediate:]
        return a @ weights["down"].T

    one_layer()  # warm
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        one_layer()
    t_layer = (time.perf_counter() - t0) / reps
    t0 = time.perf_counter()
    for _ in range(reps):
        x @ lm_w.T
    t_lm = (time.perf_counter() - t0) / reps * (s.vocab / vocab_slice)
    t_step = t_layer * layers_total + t_lm
    return {
        "value": batch / t_step,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"CPU oracle, fp32: 1 decoder layer (4 pre-dequantized int8 linears + per-row fp32 paged "
                   f"attention over the same {batch} contexts) x{reps} + lm_head on {vocab_slice}/{s.vocab} rows, "
                   f"extrapolated to {layers_total} layers + full lm_head"),
        "sec_per_step": t_step,
        "host": cpu_info(),
    }


def family_launches(model, pool, tables, seq_lens, bsz, dev) -> dict:
    """Per kernel family: (callable issuing that family's launches of one decode step, launches per call)."""
    import torch

    from runtime_amd.phase2.int8_linear import int8_linear, int8_linear_partials
    from runtime_amd.phase2.paged_attention_hip import _decode

    s = model.shape
    g = torch.Generator(device=dev).manual_seed(3)
    x_h = torch.randn(bsz, s.hidden, generator=g, device=dev).half()
    x_a = torch.randn(bsz, s.heads * s.head_dim, generator=g, device=dev).half()
    q = torch.randn(bsz, s.heads, 1, s.head_dim, generator=g, device=dev).half()
    lens = (seq_lens + 1).to(torch.int32)
    out = {}

    splits = model.buffers(bsz).splits

    def lin(name, x):
        # The call the decode step makes: split-K partials (summed by the consuming glue
        # kernel) when the shape splits, else the fused kernel writing fp16.
        outs = [torch.empty(bsz, getattr(layer, name)[2], device=dev, dtype=torch.float16) for layer in model.layers]
        part = model.buffers(bsz).part

        def run():
            for layer, y in zip(model.layers, outs):
                packed, scale, n, bias = getattr(layer, name)
                if splits[name] > 1:
                    int8_linear_partials(x, packed, scale, n, part)
                else:
                    int8_linear(x, packed, scale, bias, n, out=y)
        return run

    nl = len(model.layers)
    if model.uses_fused_qkv(bsz):
        from runtime_amd.phase2.decode_glue import qkv_linear_rope_append

        buf = model.buffers(bsz)

        def qkv_rope():
            # As the step runs it: the QKV projection with RoPE and the K/V append in its
            # epilogue (it rewrites the slots at seq_lens, which the next step writes anyway).
            for li, layer in enumerate(model.layers):
                packed, scale, _, bias = layer.qkv
                qkv_linear_rope_append(x_h, packed, scale, bias, model.rope, seq_lens, buf.q, pool.k_layer_view(li),
                                       pool.v_layer_view(li), tables, s.heads, s.kv_heads, err=buf.err)
        out["qkv"] = (qkv_rope, nl)
    else:
        out["qkv"] = (lin("qkv", x_h), nl)
    out["o"] = (lin("o", x_a), nl)
    buf = model.buffers(bsz)

    def gate_up():
        # As the step runs it: gate||up with the SwiGLU product in the epilogue.
        for layer in model.layers:
            model._gate_up(buf, layer.gate_up, bsz, None)
    out["gate_up"] = (gate_up, nl)
    out["down"] = (lin("down", buf.act), nl)

    def attn():
        for li in range(len(model.layers)):
            _decode(q, pool.k_layer_view(li), pool.v_layer_view(li), tables, lens, s.head_dim**-0.5, s.group)
    out["attn"] = (attn, nl)
    lm_y = torch.empty(bsz, s.vocab, device=dev, dtype=torch.float16)

    def lm():
        # One launch per step, repeated in its timing graph so that the graph launch is
        # amortised as for the per-layer families. Each repeat re-reads the weights from HBM:
        # they exceed the 256 MB MALL, and a sequential sweep of them leaves no reusable lines.
        packed, scale, n, bias = model.lm_head
        for _ in range(LM_HEAD_REPEATS):
            int8_linear(x_h, packed, scale, bias, n, out=lm_y)
    out["lm_head"] = (lm, LM_HEAD_REPEATS)
    return out


LM_HEAD_REPEATS = 8


def time_family(run, launches: int, reps: int) -> float:
    """Average seconds per launch of one family, from graph replays between HIP events."""
    import torch

    run()  # eager warm-up (workspaces)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(graph):
        run()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / (reps * launches)


COPY_PROBE_BYTES = 1 << 30
TRAFFIC_PROFILE = os.path.join(HERE, "profiles", "paged_attn_traffic_llama3_8b_b32.md")


def copy_bandwidth(reps: int = 10) -> dict:
    """The box's streaming rate beside the nominal peak: a 1 GiB device-to-device copy,
    HIP-event timed over ``reps`` copies; bytes = read + written."""
    import torch

    src = torch.empty(COPY_PROBE_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    t = a.elapsed_time(b) * 1e-3 / reps
    del src, dst
    torch.cuda.empty_cache()
    gbps = 2 * COPY_PROBE_BYTES / t / 1e9
    return {"gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "what": "1 GiB device-to-device copy (torch copy_), read + written bytes"}


def measured_traffic(kernel: str, model: str, batch: int):
    """HBM bytes per launch of ``kernel`` from the committed counter summary (two rocprofv3 --pmc
    passes, FETCH_SIZE and WRITE_SIZE, scaled by a 1 GiB copy), for the default workload only."""
    import re

    if model != "llama3-8b" or batch != 32 or not os.path.exists(TRAFFIC_PROFILE):
        return None
    with open(TRAFFIC_PROFILE) as f:
        m = re.search(r"^bench-traffic: kernel=(\w+) bytes_per_launch=(\d+) algorithmic_bytes=(\d+)$", f.read(), re.M)
    if not m or m.group(1) != kernel:
        return None
    return int(m.group(2)), int(m.group(3))


def traffic_probe(args) -> int:
    """Kernels for the HBM-traffic counter passes, nothing else: the bench's attention calls
    (same contexts, pool, seed; one launch per layer so no launch re-reads the previous
    one's K/V from the 256 MB MALL) and one copy of COPY_PROBE_BYTES, whose counter reading
    calibrates FETCH_SIZE / WRITE_SIZE (it reads and writes exactly that many bytes)."""
    import torch

    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.decode_step import LLAMA3_8B, QWEN2_05B, make_contexts
    from runtime_amd.phase2.paged_attention_hip import _decode
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool
    from oracle.paged_attention import attention_bytes

    _hip.load()
    dev = torch.device("cuda:0")
    shape = LLAMA3_8B if args.model == "llama3-8b" else QWEN2_05B
    n_layers = args.layers or shape.layers
    bs = 16
    headroom = args.warmup + args.steps + args.kernel_steps + 2  # the bench's table width
    lens, tables = make_contexts(args.batch, args.ctx_lo, args.ctx_hi, bs, args.pool_blocks, headroom=headroom, seed=0)
    pool = GpuKVBlockPool(num_blocks=args.pool_blocks, block_size_tokens=bs, num_layers=n_layers,
                          num_kv_heads=shape.kv_heads, head_dim=shape.head_dim, dtype=torch.float16, device=dev)
    pool._ensure_pools()
    gk = torch.Generator(device=dev).manual_seed(1)
    for t in (pool._k_pool, pool._v_pool):
        flat = t.view(-1)
        for i in range(0, flat.numel(), 1 << 28):
            flat[i:i + (1 << 28)].normal_(generator=gk)
    q = torch.randn(args.batch, shape.heads, 1, shape.head_dim, generator=gk, device=dev).half()
    tables_d = tables.to(dev)
    lens_d = (lens + 1).to(device=dev, dtype=torch.int32)
    for _ in range(args.traffic_probe):
        for li in range(n_layers):
            _decode(q, pool.k_layer_view(li), pool.v_layer_view(li), tables_d, lens_d, shape.head_dim**-0.5,
                    shape.group)
    src = torch.empty(COPY_PROBE_BYTES // 2, dtype=torch.float16, device=dev).normal_(generator=gk)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    attn_b = attention_bytes([x + 1 for x in lens.tolist()], shape.kv_heads, shape.head_dim, shape.heads, bs)
    print(json.dumps({"probe": "paged_attn", "launches": args.traffic_probe * n_layers,
                      "attn_bytes_per_launch": attn_b, "copy_bytes": COPY_PROBE_BYTES}), flush=True)
    return 0


PREFIX_GROUPS, PREFIX_TOKENS, ROTATE_EVERY = 16, 1024, 16
GRAPH_WARMUP = 2


def prefix_batch_bench(args) -> int:
    """Shared-prefix continuous batch on the native step: ``args.batch`` rows in 16 groups
    whose rows alias one 1024-token prefix (block ids shared, stored once), contexts
    U[1, 8192]. Every 16 steps the rows b with b % 8 == epoch % 8 finish and new requests
    of the same group join their slots (freed blocks reused; tables, lengths and tokens
    rewritten in place between replays of one captured step graph, all inside the timed
    region). ``value`` is tokens/s; the HBM figure counts weights + unique K/V bytes."""
    import torch

    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.decode_step import LLAMA3_8B, QWEN2_05B, Int8DecodeModel
    from runtime_amd.phase2.paged_attention_hip import _decode
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool
    from runtime_amd.phase2.prefix_batch import PrefixBatch

    _hip.load()
    dev = torch.device("cuda:0")
    shape = LLAMA3_8B if args.model == "llama3-8b" else QWEN2_05B
    n_layers = args.layers or shape.layers
    bsz, bs = args.batch, 16
    lo, hi = 1, 8192
    total_steps = args.warmup + 1 + GRAPH_WARMUP + args.steps
    num_blocks = 40960
    t_setup = time.perf_counter()
    pb = PrefixBatch(batch=bsz, groups=PREFIX_GROUPS, prefix_tokens=PREFIX_TOKENS, lo=lo, hi=hi, block_size=bs,
                     num_blocks=num_blocks, headroom=total_steps + ROTATE_EVERY, seed=0)
    model = Int8DecodeModel(shape, device=dev, seed=0, layers=n_layers)
    model.shared_kv_blocks = not args.stream_shared_kv  # rows of a group alias the prefix blocks
    pool = GpuKVBlockPool(num_blocks=num_blocks, block_size_tokens=bs, num_layers=n_layers,
                          num_kv_heads=shape.kv_heads, head_dim=shape.head_dim, dtype=torch.float16, device=dev)
    pool._ensure_pools()
    gk = torch.Generator(device=dev).manual_seed(1)
    for t in (pool._k_pool, pool._v_pool):
        flat = t.view(-1)
        for i in range(0, flat.numel(), 1 << 28):
            flat[i:i + (1 << 28)].normal_(generator=gk)
    tables_d = torch.zeros(bsz, pb.max_blocks, dtype=torch.int32, device=dev)
    seq_lens = torch.zeros(bsz, dtype=torch.int32, device=dev)
    pb.upload(tables_d, seq_lens)
    gt = torch.Generator().manual_seed(2)
    tokens = torch.randint(0, shape.vocab, (bsz,), generator=gt).to(dev)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    def step():
        model.step(tokens, pool, tables_d, seq_lens, out=tokens)

    for _ in range(args.warmup):
        step()
        pb.advance(1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    pb.advance(1)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()  # recorded, not run: the lengths do not advance
    for _ in range(GRAPH_WARMUP):  # the first replays of a new graph carry one-time costs
        graph.replay()
        pb.advance(1)
    torch.cuda.synchronize()
    assert seq_lens.cpu().tolist() == pb.lens.tolist(), "device lengths diverged from the schedule"

    kv_token_bytes = n_layers * shape.kv_heads * shape.head_dim * 2 * 2  # K and V, every layer

    def rotation(k: int) -> list[int]:
        """Rows that finish before step k (every ROTATE_EVERY steps, one row in 8)."""
        if k == 0 or k % ROTATE_EVERY:
            return []
        return [b for b in range(bsz) if b % 8 == (k // ROTATE_EVERY) % 8]

    # Timed: the step graph plus the join/finish work (host schedule, table and length
    # uploads, new tokens) every ROTATE_EVERY steps.
    rotated = 0
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for k in range(args.steps):
        rows = rotation(k)
        if rows:
            pb.rotate(rows)
            pb.upload_rows(rows, tables_d, seq_lens)
            tokens[rows] = torch.randint(0, shape.vocab, (len(rows),), generator=gt).to(dev)
            rotated += len(rows)
        graph.replay()
        pb.advance(1)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    assert seq_lens.cpu().tolist() == pb.lens.tolist(), "device lengths diverged from the schedule"

    # Byte accounting, outside the timed region: the same seeded host schedule replayed on the
    # CPU, counting each step's K/V tokens read (logical) and stored (unique).
    acct = PrefixBatch(batch=bsz, groups=PREFIX_GROUPS, prefix_tokens=PREFIX_TOKENS, lo=lo, hi=hi, block_size=bs,
                       num_blocks=num_blocks, headroom=total_steps + ROTATE_EVERY, seed=0)
    acct.advance(args.warmup + 1 + GRAPH_WARMUP)
    uniq, logical = [], []
    for k in range(args.steps):
        rows = rotation(k)
        if rows:
            acct.rotate(rows)
        uniq.append(acct.unique_tokens(1))
        logical.append(acct.logical_tokens(1))
        acct.advance(1)
    assert acct.lens.tolist() == pb.lens.tolist()

    # Attention family at the final state (32 launches per step, one graph), as in the headline bench.
    s_ = model.shape
    q = torch.randn(bsz, s_.heads, 1, s_.head_dim, generator=gk, device=dev).half()
    lens_attn = (seq_lens + 1).to(torch.int32)

    def attn():
        for li in range(n_layers):
            _decode(q, pool.k_layer_view(li), pool.v_layer_view(li), tables_d, lens_attn, s_.head_dim**-0.5, s_.group,
                    shared_blocks=model.shared_kv_blocks)
    attn_s = time_family(attn, n_layers, args.kernel_steps)
    # One attention launch (one layer) reads these K/V bytes at the final state.
    final_uniq = pb.unique_tokens(1) * shape.kv_heads * shape.head_dim * 2 * 2
    final_logical = pb.logical_tokens(1) * shape.kv_heads * shape.head_dim * 2 * 2

    lin = model.linear_bytes(bsz)
    weight_bytes = n_layers * (lin["qkv"] + lin["o"] + lin["gate_up"] + lin["down"]) + lin["lm_head"]
    uniq_b = sum(uniq) / len(uniq) * kv_token_bytes
    logical_b = sum(logical) / len(logical) * kv_token_bytes
    value = bsz / (ms * 1e-3)
    out = {
        "metric": "decode tokens/sec + achieved HBM GB/s (% peak), int8-W linear + paged-attn",
        "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "w8a16 (int8 weights, fp16 activations/KV, fp32 accumulate)",
        "data": "synthetic (random-init weights quantized on device, random K/V)",
        "config": {
            "workload": f"{args.model}-shaped int8 decode step, {bsz} rows in {PREFIX_GROUPS} groups sharing a "
                        f"{PREFIX_TOKENS}-token prefix (aliased blocks), contexts U[{lo},{hi}], {bsz // 8} rows "
                        f"finish and join every {ROTATE_EVERY} steps",
            "batch": bsz, "layers": n_layers, "block_size": bs, "pool_blocks": num_blocks, "hip_graph": True,
            "parallelism": "none (1 GPU)", "rows_rotated": rotated,
        },
        "kv_logical_bytes_per_step": int(logical_b), "kv_unique_bytes_per_step": int(uniq_b),
        "weight_bytes_per_step": weight_bytes,
        "step_gbps_unique": round((weight_bytes + uniq_b) / (ms * 1e-3) / 1e9, 1),
        "step_hbm_frac_unique": round((weight_bytes + uniq_b) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "attn": {"avg_us": round(attn_s * 1e6, 2), "unique_bytes": final_uniq, "logical_bytes": final_logical,
                 "gbps_unique": round(final_uniq / attn_s / 1e9, 1),
                 "gbps_logical": round(final_logical / attn_s / 1e9, 1)},
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(out), flush=True)
    return 0


def graph_time(run, launches: int, reps: int = 4) -> float:
    """Seconds per launch of ``run`` (``launches`` kernel calls), captured once and replayed."""
    import torch

    run()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / (reps * launches)


def linear_sweep_bench(args) -> int:
    """Config 1 (x [1, 4096] @ W [4096, 4096], seed 0) and config 4 (the Llama-3-8B projections,
    seed 1000 + shape index, M in {1, 8, 32, 64}) through ``int8_linear``. Weights are
    N(0, 0.02) quantized on the device; each timed graph walks over enough distinct weight
    copies (> 512 MB) that no launch reads its weights from the 256 MB MALL. Bytes are the
    algorithmic N*K + 2N + 2MK + 2MN. The CPU oracle (fp32, pre-dequantized weights and with
    the dequantization per call) is timed on config 1."""
    import numpy as np
    import torch

    from oracle import int8_quant
    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.int8_linear import int8_linear, pack_weight, quantize_weight

    _hip.load()
    dev = torch.device("cuda:0")
    shapes = [("config1", 4096, 4096, [1])] + [(n, k, nn, [1, 8, 32, 64]) for n, k, nn in
                                               (("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 28672),
                                                ("down", 14336, 4096))]
    rows = []
    for idx, (name, k, n, ms) in enumerate(shapes):
        g = torch.Generator(device=dev).manual_seed(0 if name == "config1" else 1000 + idx - 1)
        copies = max(4, math.ceil(600e6 / (n * k)))
        weights = []
        for _ in range(copies):
            q, sc = quantize_weight(torch.randn(n, k, generator=g, device=dev) * 0.02)
            weights.append((pack_weight(q), sc))
        for m in ms:
            x = torch.randn(m, k, generator=g, device=dev).half()
            y = torch.empty(m, n, dtype=torch.float16, device=dev)

            def run():
                for packed, sc in weights:
                    int8_linear(x, packed, sc, None, n, out=y)
            t = graph_time(run, copies)
            byts = n * k + 2 * n + 2 * m * k + 2 * m * n
            rows.append({"shape": name, "m": m, "n": n, "k": k, "avg_us": round(t * 1e6, 2),
                         "gbps": round(byts / t / 1e9, 1), "frac": round(byts / t / 1e9 / HBM_PEAK_GBPS, 4)})
            print(f"[linear] {name} M={m}: {t * 1e6:.2f} us, {byts / t / 1e9:.1f} GB/s", file=sys.stderr, flush=True)
        del weights
        torch.cuda.empty_cache()
    # CPU oracle on config 1.
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    q, sc = int8_quant.quantize_per_channel(w)
    xh = rng.standard_normal((1, 4096)).astype(np.float16)
    wd = torch.from_numpy(int8_quant.dequantize(q, sc))
    xf = torch.from_numpy(xh.astype(np.float32))
    qt, st = torch.from_numpy(q), torch.from_numpy(sc.astype(np.float32))
    reps = 200
    t0 = time.perf_counter()
    for _ in range(reps):
        xf @ wd.T
    t_pre = (time.perf_counter() - t0) / reps
    t0 = time.perf_counter()
    for _ in range(20):
        xf @ (qt.float() * st[:, None]).T
    t_deq = (time.perf_counter() - t0) / 20
    c1 = rows[0]
    byts1 = 4096 * 4096 + 2 * 4096 + 2 * 4096 + 2 * 4096
    out = {
        "metric": "int8 linear algorithmic HBM GB/s (config 1; config 4 sweep in 'sweep')",
        "value": c1["gbps"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "w8a16 (int8 weights, fp16 activations, fp32 accumulate)",
        "data": "synthetic (N(0,0.02) weights quantized on device)",
        "config": {"workload": "int8 linear: 4096x4096 at M=1 (config 1); Llama-3-8B qkv/o/gate_up/down at "
                               "M in {1,8,32,64} (config 4)"},
        "roofline": {"bound": "hbm", "kernel": "config1", "achieved": c1["gbps"], "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": c1["frac"], "traffic": None},
        "sweep": rows,
        "cpu_baseline": {"value": round(byts1 / t_pre / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
                         "sample": "config 1 on the CPU oracle (fp32 x @ dequantized W^T, weights dequantized "
                                   "once); with the dequantization in each call: "
                                   f"{byts1 / t_deq / 1e9:.2f} GB/s",
                         "us_per_call": round(t_pre * 1e6, 1), "us_per_call_dequant": round(t_deq * 1e6, 1)},
    }
    print(json.dumps(out), flush=True)
    return 0


def attention_bench(args) -> int:
    """Config 2: ``torch.manual_seed(0)``; seq_lens ~ U{128..4096} for 32 rows; each row takes
    ceil(S/16) ids from one randperm(16384); q [32, 32, 1, 128] and K/V N(0, 1) fp16; scale
    1/sqrt(128). The timed graph walks over 32 layer copies of the pool (one call per layer,
    as in the decode step) so no call re-reads K/V from the MALL. The CPU oracle (per-row fp32
    paged attention) is timed on the same inputs."""
    import torch

    from oracle.paged_attention import attention_bytes, decode_rows_fp32
    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.paged_attention_hip import _decode
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    _hip.load()
    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, bs, nb, L = 32, 32, 8, 128, 16, 16384, 32
    torch.manual_seed(0)
    lens = torch.randint(128, 4097, (B,))
    perm = torch.randperm(nb)
    nblk = [math.ceil(int(x) / bs) for x in lens]
    tables = torch.zeros(B, max(nblk), dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        tables[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    q = torch.randn(B, Hq, 1, D).half()
    pool = GpuKVBlockPool(num_blocks=nb, block_size_tokens=bs, num_layers=L, num_kv_heads=Hkv, head_dim=D,
                          dtype=torch.float16, device=dev)
    pool._ensure_pools()
    gk = torch.Generator(device=dev).manual_seed(0)
    for t in (pool._k_pool, pool._v_pool):
        flat = t.view(-1)
        for i in range(0, flat.numel(), 1 << 28):
            flat[i:i + (1 << 28)].normal_(generator=gk)
    qd, td, ld = q.to(dev), tables.to(dev), lens.to(device=dev, dtype=torch.int32)
    scale = D**-0.5

    def run():
        for li in range(L):
            _decode(qd, pool.k_layer_view(li), pool.v_layer_view(li), td, ld, scale, Hq // Hkv)
    t = graph_time(run, L, reps=max(2, args.kernel_steps))
    byts = attention_bytes(lens.tolist(), Hkv, D, Hq, bs)
    # CPU oracle on layer 0's blocks.
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ids = torch.unique(tables[tables >= 0])
    kc = pool.k_layer_view(0)[ids.to(dev)].cpu()
    vc = pool.v_layer_view(0)[ids.to(dev)].cpu()
    remap = torch.full((nb,), -1, dtype=torch.int32)
    remap[ids] = torch.arange(ids.numel(), dtype=torch.int32)
    tc = remap[tables.long()]
    decode_rows_fp32(q, kc, vc, tc, lens.tolist(), scale, Hq // Hkv)  # warm
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        decode_rows_fp32(q, kc, vc, tc, lens.tolist(), scale, Hq // Hkv)
    t_cpu = (time.perf_counter() - t0) / reps
    achieved = byts / t / 1e9
    out = {
        "metric": "paged decode attention algorithmic HBM GB/s (config 2)", "value": round(achieved, 1),
        "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "avg_us": round(t * 1e6, 2),
        "dtype": "fp16 K/V and q, fp32 softmax and accumulation",
        "data": "synthetic (N(0,1) K/V, q; torch.manual_seed(0) contexts and block ids)",
        "config": {"workload": "paged decode attention, B 32, Hq 32, Hkv 8, D 128, block 16, contexts "
                               "U[128,4096], pool 16384 blocks x 32 layers", "bytes_per_call": byts},
        "roofline": {"bound": "hbm", "kernel": "attn", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None},
        "hbm_copy": copy_bandwidth(),
        "cpu_baseline": {"value": round(byts / t_cpu / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
                         "sample": "one call of the per-row fp32 oracle (oracle.paged_attention.decode_rows_fp32) "
                                   "on the same inputs", "ms_per_call": round(t_cpu * 1e3, 1)},
    }
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards without exchange; see the design notes). Run with --gpus 1.", file=sys.stderr)
        return 2

    if args.traffic_probe:
        return traffic_probe(args)
    if args.workload == "prefix-batch":
        return prefix_batch_bench(args)
    if args.workload == "linear-sweep":
        return linear_sweep_bench(args)
    if args.workload == "attention":
        return attention_bench(args)

    import torch

    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.decode_step import LLAMA3_8B, QWEN2_05B, Int8DecodeModel, make_contexts
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool
    from oracle.paged_attention import attention_bytes

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    _hip.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    shape = LLAMA3_8B if args.model == "llama3-8b" else QWEN2_05B
    n_layers = args.layers or shape.layers
    bsz = args.batch
    bs = 16
    total_steps = args.warmup + 1 + GRAPH_WARMUP + args.steps + args.kernel_steps + 2
    lens, tables = make_contexts(bsz, args.ctx_lo, args.ctx_hi, bs, args.pool_blocks, headroom=total_steps, seed=0)
    t_setup = time.perf_counter()
    model = Int8DecodeModel(shape, device=dev, seed=0, layers=n_layers)
    pool = GpuKVBlockPool(num_blocks=args.pool_blocks, block_size_tokens=bs, num_layers=n_layers,
                          num_kv_heads=shape.kv_heads, head_dim=shape.head_dim, dtype=torch.float16, device=dev)
    pool._ensure_pools()
    gk = torch.Generator(device=dev).manual_seed(1)
    for t in (pool._k_pool, pool._v_pool):
        flat = t.view(-1)
        chunk = 1 << 28
        for i in range(0, flat.numel(), chunk):
            flat[i:i + chunk].normal_(generator=gk)
    tables_d = tables.to(dev)
    seq_lens = lens.to(dev).clone()
    tokens = torch.randint(0, shape.vocab, (bsz,), generator=torch.Generator().manual_seed(2)).to(dev)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    def step():
        model.step(tokens, pool, tables_d, seq_lens, out=tokens)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    graph = None
    if not args.no_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()  # one more eager step on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(GRAPH_WARMUP):  # untimed: the first replays of a new graph carry one-time costs
            graph.replay()
        torch.cuda.synchronize()

    lens_before = seq_lens.cpu().tolist()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    lens_after = seq_lens.cpu().tolist()

    # Per-kernel durations. Each family's launches of one step (e.g. the 32 paged
    # decode calls, one per layer, on the same inputs the step uses) are captured
    # into their own graph and replayed back-to-back between two HIP events on
    # the current stream, so host launch latency never lands inside the interval.
    kdur = {name: time_family(run, launches, args.kernel_steps)
            for name, (run, launches) in family_launches(model, pool, tables_d, seq_lens, bsz, dev).items()}

    # Algorithmic bytes.
    lin = model.linear_bytes(bsz)
    mid_lens = [(a + b) / 2 + 1 for a, b in zip(lens_before, lens_after)]
    attn_b = attention_bytes([round(x) for x in mid_lens], shape.kv_heads, shape.head_dim, shape.heads, bs)
    append_b = 2 * bsz * shape.kv_heads * shape.head_dim * 2
    step_bytes = n_layers * (lin["qkv"] + lin["o"] + lin["gate_up"] + lin["down"] + attn_b + append_b) + lin["lm_head"]
    step_bytes += bsz * shape.hidden * 2
    # The family graphs ran after the timed steps, at contexts lens_after (+1 token).
    attn_kernel_b = attention_bytes([x + 1 for x in lens_after], shape.kv_heads, shape.head_dim, shape.heads, bs)
    per_launch = {"attn": attn_kernel_b, **lin}
    per_step = {k: (n_layers if k != "lm_head" else 1) for k in kdur}
    dominant = max(kdur, key=lambda k: kdur[k] * per_step[k])
    avg = kdur[dominant]
    achieved = per_launch[dominant] / avg / 1e9
    kernels = {k: {"avg_us": round(kdur[k] * 1e6, 2), "launches_per_step": per_step[k],
                   "bytes_per_launch": per_launch[k], "gbps": round(per_launch[k] / kdur[k] / 1e9, 1),
                   "frac": round(per_launch[k] / kdur[k] / 1e9 / HBM_PEAK_GBPS, 4)} for k in kdur}

    value = bsz / (ms * 1e-3)
    traffic = measured_traffic(dominant, args.model, bsz) if n_layers == shape.layers else None
    out = {
        "metric": "decode tokens/sec + achieved HBM GB/s (% peak), int8-W linear + paged-attn",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w8a16 (int8 weights, fp16 activations/KV, fp32 accumulate)",
        "data": "synthetic (random-init weights quantized on device, random K/V)",
        "config": {
            "workload": f"{args.model}-shaped int8 decode step (int8 linears + paged-attn decode), batch {bsz}",
            "batch": bsz, "layers": n_layers, "hidden": shape.hidden, "heads": shape.heads,
            "kv_heads": shape.kv_heads, "head_dim": shape.head_dim, "intermediate": shape.intermediate,
            "vocab": shape.vocab, "contexts": f"U[{args.ctx_lo},{args.ctx_hi}] seed 0", "block_size": bs,
            "pool_blocks": args.pool_blocks, "hip_graph": graph is not None, "parallelism": "none (1 GPU)",
        },
        "step_hbm_bytes": step_bytes,
        "step_gbps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "step_hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic[0] if traffic else None,
                     "traffic_note": (f"HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE "
                                      f"(copy-calibrated), profiles/{os.path.basename(TRAFFIC_PROFILE)}; "
                                      f"{traffic[1]} algorithmic bytes at that run's contexts") if traffic else None},
        "kernels": kernels,
        "hbm_copy": copy_bandwidth(),
        "setup_s": round(setup_s, 1),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(shape, bsz, lens.tolist(), n_layers)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
