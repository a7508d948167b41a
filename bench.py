"""Decode-step benchmark on one MI355X: int8 (W8A16) linears + paged-attention decode.

Headline workload (the benchmark's north star): a Llama-3-8B-shaped int8 weight-only decoder
(32 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, intermediate 14336, vocab 128256),
batch 32, one token per row per step, paged fp16 KV with block_size 16 in a 16384-block pool,
contexts ~ U[128, 4096] drawn with seed 0 (config-2-like), block tables from one randperm of
the pool. Weights are random N(0, 0.02) quantized on the device with the build's int8 format;
K/V and embeddings are random. Inputs are resident in HBM before timing starts.

Prints ONE JSON line. ``value`` = decode tokens/s of the whole step (B tokens per step), timed
over ``--steps`` HIP-graph replays of the step after ``--warmup`` eager steps, the capture and
2 untimed replays. ``kernels`` holds each kernel family's average launch duration: that
family's launches of one step (same inputs, same stream) are captured into their own graph
and replayed ``--kernel-steps`` times back-to-back between two HIP events, so no host launch
latency lands inside the interval (the single lm_head launch is repeated 8 times in its graph).
``roofline`` is for the family with the most time per step. ``cpu_baseline`` times the CPU
oracle on a bounded sample (one decoder layer at the same batch and contexts, plus an lm_head
slice), extrapolated to the full step. ``hbm_copy`` is a timed 1 GiB device-to-device copy.

``configs`` carries every other benchmark configuration in the same run, each with its
algorithmic bytes, achieved GB/s, roofline fraction and (where the configuration asks for one) a
CPU baseline:

* ``config1_linear`` and ``config4_linear_sweep``: the single 4096x4096 int8 linear at M=1 and
  the Llama-3-8B projections at M in {1, 8, 32, 64}, each timed over enough distinct weight
  copies (> 512 MB) that no launch reads its weights from the 256 MB MALL;
* ``config2_attention``: one paged decode call on config 2's inputs (torch.manual_seed(0)
  contexts and block ids), timed over the 32 layers of the headline pool, plus the gather
  ceiling: the same K/V reads without the math (``mx_kv_gather_probe``), in the decode
  kernel's own pattern and with whole blocks per workgroup;
* ``config3_qwen2_0.5b``: the Qwen2-0.5B-shaped step at batch 16, contexts U[512, 2048];
* ``config5_prefix_batch``: 128 rows in 16 groups of 8 aliasing a 1024-token prefix, contexts
  U[1, 8192], 16 rows finishing and 16 joining every 16 steps, on the headline model.

``--workload`` runs one of them alone (for profiling); ``--traffic-probe`` runs only the
kernels of a counter pass.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "llm-serving-runtime_amd"))
sys.path.insert(0, HERE)

HBM_PEAK_GBPS = 8000.0
METRIC = "decode tokens/sec + achieved HBM GB/s (% peak), int8-W linear + paged-attn"
DTYPE = "w8a16 (int8 weights, fp16 activations/KV, fp32 accumulate)"
DATA = "synthetic (random-init weights quantized on device, random K/V)"
GRAPH_WARMUP = 2
LM_HEAD_REPEATS = 8
COPY_PROBE_BYTES = 1 << 30
ATTN_TRAFFIC_PROFILE = os.path.join(HERE, "profiles", "paged_attn_traffic_llama3_8b_b32.md")
GEMM_COUNTER_PROFILE = os.path.join(HERE, "profiles", "int8_gemm_counters_llama3_8b_b32.md")
SWEEP_COUNTER_PROFILE = os.path.join(HERE, "profiles", "int8_linear_sweep_counters_configs1_4.md")
PREFIX_GROUPS, PREFIX_TOKENS, ROTATE_EVERY = 16, 1024, 16


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=None, help="rows (default 32; 128 for --workload prefix-batch)")
    ap.add_argument("--workload", choices=["all", "decode", "prefix-batch", "linear-sweep", "attention", "qwen",
                                           "probes"],
                    default="all",
                    help="all: the headline step with every config in 'configs' (default). decode: the headline "
                         "step alone. prefix-batch: config 5. linear-sweep: configs 1 and 4. attention: config 2 "
                         "and the gather ceiling. qwen: config 3")
    ap.add_argument("--model", choices=["llama3-8b", "qwen2-0.5b"], default="llama3-8b")
    ap.add_argument("--layers", type=int, default=None, help="override layer count (diagnostics only)")
    ap.add_argument("--ctx-lo", type=int, default=128)
    ap.add_argument("--ctx-hi", type=int, default=4096)
    ap.add_argument("--pool-blocks", type=int, default=16384)
    ap.add_argument("--kernel-steps", type=int, default=5, help="graph replays per kernel family for kernel timing")
    ap.add_argument("--prefix-steps", type=int, default=40, help="timed steps of config 5")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--fuse-mlp", action="store_true",
                    help="run gate||up and down as one launch where the shape takes it (Int8DecodeModel.fuse_mlp)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-probe", type=int, default=0, metavar="REPS",
                    help="instead of the bench: REPS rounds of one kernel family's launches of the headline step "
                         "and a 1 GiB copy, for rocprofv3 --pmc passes (see --probe-family)")
    ap.add_argument("--probe-family", choices=["attn", "linears", "sweep"], default="attn",
                    help="attn / linears: the headline step's attention or its four projections; sweep: "
                         "int8_linear alone on config 4's shapes (and config 1's at --batch 1) at M = --batch")
    ap.add_argument("--kv-layout", choices=["split", "interleaved"], default="interleaved",
                    help="KV pool layout (GpuKVBlockPool kv_layout) of the headline, config 2 and config 5 pools")
    ap.add_argument("--stream-shared-kv", action="store_true",
                    help="config 5: read the aliased K/V with streaming loads (no MX_PA_SHARED_BLOCKS)")
    args = ap.parse_args()
    if args.batch is None:
        args.batch = 128 if args.workload == "prefix-batch" else 32
    return args


# ---------------------------------------------------------------------------------------------
# Shared helpers
# ---------------------------------------------------------------------------------------------
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


def frac(gbps: float) -> float:
    return round(gbps / HBM_PEAK_GBPS, 4)


def graph_time(run, launches: int, reps: int = 4) -> float:
    """Seconds per launch of ``run`` (``launches`` kernel calls): captured once into a HIP graph,
    replayed ``reps`` times back-to-back between two HIP events on the current stream."""
    import torch

    run()  # eager warm-up (workspaces)
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
    return {"gbps": round(gbps, 1), "frac": frac(gbps), "what": "1 GiB device-to-device copy (torch copy_), "
                                                                "read + written bytes"}


def committed_figures(path: str, prefix: str) -> dict[str, dict]:
    """``prefix: key=value ...`` lines of a committed profile summary, keyed by ``kernel``."""
    if not os.path.exists(path):
        return {}
    out = {}
    with open(path) as f:
        for m in re.finditer(rf"^{prefix}: (.*)$", f.read(), re.M):
            kv = dict(item.split("=", 1) for item in m.group(1).split())
            out[kv.pop("kernel")] = {k: (float(v) if re.fullmatch(r"[-+0-9.eE]+", v) else v) for k, v in kv.items()}
    return out


def fill_normal(t, gen) -> None:
    """N(0, 1) in place, one leading slice at a time (the pool tensors may be strided views)."""
    for i in range(t.shape[0]):
        t[i].normal_(generator=gen)


CPU_SAMPLE_S = 10.0  # seconds of CPU work per baseline sample (a bounded sample of the workload)


def repeat_for(fn, seconds: float, min_reps: int = 3) -> tuple[float, int]:
    """Mean seconds per call of ``fn`` over as many calls as fit in ``seconds`` (at least ``min_reps``)."""
    n, t0 = 0, time.perf_counter()
    while n < min_reps or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def cpu_step_baseline(shape, batch: int, lens, layers_total: int) -> dict:
    """The CPU oracle on one decoder layer (the four linears on pre-dequantized fp32 weights and
    per-row fp32 paged attention over the same contexts) and an lm_head slice, extrapolated to the
    full step."""
    import numpy as np
    import torch

    from oracle import int8_quant, paged_attention

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rng = np.random.default_rng(0)
    s = shape
    mats = {"qkv": (s.qkv_out, s.hidden), "o": (s.hidden, s.heads * s.head_dim),
            "gate_up": (2 * s.intermediate, s.hidden), "down": (s.hidden, s.intermediate)}
    weights = {}
    for name, (n, k) in mats.items():
        q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        sc = (np.abs(rng.standard_normal(n)) * 1e-3 + 1e-4).astype(np.float16)
        weights[name] = torch.from_numpy(int8_quant.dequantize(q, sc))
    vocab_slice = min(16384, s.vocab)
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
        x @ weights["qkv"].T
        attn = paged_attention.decode_rows_fp32(q, k_layer, v_layer, tables, lens, s.head_dim**-0.5, s.group)
        attn.reshape(batch, -1) @ weights["o"].T
        gu = x @ weights["gate_up"].T
        a = torch.nn.functional.silu(gu[:, :s.intermediate]) * gu[:, s.intermediate:]
        return a @ weights["down"].T

    one_layer()  # warm
    t_layer, n_layer = repeat_for(one_layer, CPU_SAMPLE_S)
    t_lm, n_lm = repeat_for(lambda: x @ lm_w.T, CPU_SAMPLE_S / 10)
    t_lm *= s.vocab / vocab_slice
    t_step = t_layer * layers_total + t_lm
    return {
        "value": round(batch / t_step, 3), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"CPU oracle, fp32: 1 decoder layer (4 pre-dequantized int8 linears + per-row fp32 paged "
                   f"attention over the same {batch} contexts) x{n_layer} + lm_head on {vocab_slice}/{s.vocab} rows "
                   f"x{n_lm}, extrapolated to {layers_total} layers + full lm_head"),
        "sec_per_step": round(t_step, 4),
        "sample_seconds": round(t_layer * n_layer + t_lm * vocab_slice / s.vocab * n_lm, 2),
        "host": cpu_info(),
    }


def time_step(step, steps: int, warmup: int, use_graph: bool = True):
    """Milliseconds per call of ``step`` over ``steps`` HIP-graph replays (after ``warmup`` eager
    calls, one eager call on the capture stream, the capture and GRAPH_WARMUP untimed replays)."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    graph = None
    if use_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(GRAPH_WARMUP):
            graph.replay()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay() if graph is not None else step()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


class Decoder:
    """A random-init int8 decoder, its paged pool (random K/V) and a batch of seeded contexts."""

    def __init__(self, shape, batch: int, lo: int, hi: int, pool_blocks: int, headroom: int, layers=None, seed=0,
                 kv_layout: str = "interleaved", fuse_mlp: bool = False):
        import torch

        from runtime_amd.phase2.decode_step import Int8DecodeModel, make_contexts
        from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

        self.dev = torch.device("cuda:0")
        self.shape, self.batch, self.bs = shape, batch, 16
        self.n_layers = layers or shape.layers
        t0 = time.perf_counter()
        self.lens, self.tables = make_contexts(batch, lo, hi, self.bs, pool_blocks, headroom=headroom, seed=seed)
        self.model = Int8DecodeModel(shape, device=self.dev, seed=seed, layers=self.n_layers)
        self.model.fuse_mlp = fuse_mlp
        self.pool = GpuKVBlockPool(num_blocks=pool_blocks, block_size_tokens=self.bs, num_layers=self.n_layers,
                                   num_kv_heads=shape.kv_heads, head_dim=shape.head_dim, dtype=torch.float16,
                                   device=self.dev, kv_layout=kv_layout)
        self.pool._ensure_pools()
        gk = torch.Generator(device=self.dev).manual_seed(seed + 1)
        fill_normal(self.pool._k_pool, gk)
        fill_normal(self.pool._v_pool, gk)
        self.tables_d = self.tables.to(self.dev)
        self.seq_lens = self.lens.to(self.dev).clone()
        self.tokens = torch.randint(0, shape.vocab, (batch,), generator=torch.Generator().manual_seed(seed + 2)
                                    ).to(self.dev)
        torch.cuda.synchronize()
        self.setup_s = time.perf_counter() - t0

    def step(self):
        self.model.step(self.tokens, self.pool, self.tables_d, self.seq_lens, out=self.tokens)

    def step_bytes(self, lens_before, lens_after) -> int:
        from runtime_amd.phase2.roofline import attention_hbm_bytes

        s, lin = self.shape, self.model.linear_bytes(self.batch)
        mid = [round((a + b) / 2 + 1) for a, b in zip(lens_before, lens_after)]
        attn_b = attention_hbm_bytes(mid, s.kv_heads, s.head_dim, s.heads, self.bs)
        append_b = 2 * self.batch * s.kv_heads * s.head_dim * 2
        return (self.n_layers * (lin["qkv"] + lin["o"] + lin["gate_up"] + lin["down"] + attn_b + append_b)
                + lin["lm_head"] + self.batch * s.hidden * 2)


# ---------------------------------------------------------------------------------------------
# Headline: the Llama-3-8B-shaped step at batch 32
# ---------------------------------------------------------------------------------------------
def family_launches(d: Decoder) -> dict:
    """Per kernel family: (callable issuing that family's launches of one decode step, launches per call)."""
    import torch

    from runtime_amd.phase2.decode_glue import qkv_linear_rope_append
    from runtime_amd.phase2.int8_linear import int8_linear, int8_linear_partials, int8_mlp_fused_partials
    from runtime_amd.phase2.paged_attention_hip import MX_PA_PLAN_READ, MX_PA_PLAN_WRITE, _decode

    model, pool, bsz, dev, s = d.model, d.pool, d.batch, d.dev, d.shape
    g = torch.Generator(device=dev).manual_seed(3)
    x_h = torch.randn(bsz, s.hidden, generator=g, device=dev).half()
    x_a = torch.randn(bsz, s.heads * s.head_dim, generator=g, device=dev).half()
    q = torch.randn(bsz, s.heads, 1, s.head_dim, generator=g, device=dev).half()
    lens = (d.seq_lens + 1).to(torch.int32)
    buf = model.buffers(bsz)
    splits = buf.splits
    out = {}

    def lin(name, x):
        # The call the step makes: split-K partials (summed by the consuming glue kernel) when the
        # shape splits, else the kernel writing fp16.
        ys = [torch.empty(bsz, getattr(layer, name)[2], device=dev, dtype=torch.float16) for layer in model.layers]

        def run():
            for layer, y in zip(model.layers, ys):
                packed, scale, n, bias = getattr(layer, name)
                if splits[name] > 1:
                    int8_linear_partials(x, packed, scale, n, buf.part)
                else:
                    int8_linear(x, packed, scale, bias, n, out=y)
        return run

    nl = len(model.layers)
    if model.uses_fused_qkv(bsz):
        def qkv_rope():
            # As the step runs it: the QKV projection with RoPE and the K/V append in its epilogue
            # (it rewrites the slots at seq_lens, which the next step writes anyway).
            for li, layer in enumerate(model.layers):
                packed, scale, _, bias = layer.qkv
                qkv_linear_rope_append(x_h, packed, scale, bias, model.rope, d.seq_lens, buf.q, pool.k_layer_view(li),
                                       pool.v_layer_view(li), d.tables_d, s.heads, s.kv_heads, err=buf.err)
        out["qkv"] = (qkv_rope, nl)
    else:
        out["qkv"] = (lin("qkv", x_h), nl)
    out["o"] = (lin("o", x_a), nl)

    def gate_up():
        for layer in model.layers:
            model._gate_up(buf, layer.gate_up, bsz, None)
    out["gate_up"] = (gate_up, nl)
    out["down"] = (lin("down", buf.act), nl)
    if model.fuse_mlp and buf.mlp_fused:
        def mlp():
            # As the step runs it at this batch: gate||up and down's split partials in one launch.
            for layer in model.layers:
                int8_mlp_fused_partials(x_h, layer.gate_up, layer.down, buf.act, buf.part, buf.mlp_sync)
        out["mlp"] = (mlp, nl)

    # As the step calls it: layer 0 records the tile plan, the later layers start from it.
    planned = model.attn_plan and not model.shared_kv_blocks and pool.block_size_tokens >= 16

    def attn():
        for li in range(nl):
            plan = (MX_PA_PLAN_WRITE if li == 0 else MX_PA_PLAN_READ) if planned else 0
            _decode(q, pool.k_layer_view(li), pool.v_layer_view(li), d.tables_d, lens, s.head_dim**-0.5, s.group,
                    plan=plan)
    out["attn"] = (attn, nl)
    lm_y = torch.empty(bsz, s.vocab, device=dev, dtype=torch.float16)

    def lm():
        # One launch per step, repeated in its graph so that the graph launch is amortised as for the
        # per-layer families; each repeat re-reads the weights from HBM (they exceed the MALL).
        packed, scale, n, bias = model.lm_head
        for _ in range(LM_HEAD_REPEATS):
            int8_linear(x_h, packed, scale, bias, n, out=lm_y)
    out["lm_head"] = (lm, LM_HEAD_REPEATS)
    return out


def family_table(d: Decoder, args, lens_after) -> tuple[dict, dict, dict, dict]:
    """Per kernel family of the step: seconds per launch (graph replays of that family's launches
    alone, run after the timed steps, so at contexts ``lens_after`` + 1), algorithmic bytes per
    launch, launches per step, and the JSON entries."""
    from runtime_amd.phase2.roofline import attention_hbm_bytes

    s = d.shape
    fams = family_launches(d)
    if "mlp" in fams:  # the step runs gate||up and down as one launch: time that, not the two apart
        del fams["gate_up"], fams["down"]
    kdur = {name: graph_time(run, launches, args.kernel_steps) for name, (run, launches) in fams.items()}
    lin = d.model.linear_bytes(d.batch)
    per_launch = {"attn": attention_hbm_bytes([x + 1 for x in lens_after], s.kv_heads, s.head_dim, s.heads, d.bs),
                  **lin, "mlp": lin["gate_up"] + lin["down"]}
    per_step = {k: (d.n_layers if k != "lm_head" else 1) for k in kdur}
    kernels = {}
    for k in kdur:
        gbps = per_launch[k] / kdur[k] / 1e9
        kernels[k] = {"avg_us": round(kdur[k] * 1e6, 2), "launches_per_step": per_step[k],
                      "bytes_per_launch": per_launch[k], "gbps": round(gbps, 1), "frac": frac(gbps)}
    return kdur, per_launch, per_step, kernels


def headline(args, d: Decoder) -> dict:
    s, bsz = d.shape, d.batch
    lens_before = d.seq_lens.cpu().tolist()
    ms = time_step(d.step, args.steps, args.warmup, use_graph=not args.no_graph)
    lens_after = d.seq_lens.cpu().tolist()
    kdur, per_launch, per_step, kernels = family_table(d, args, lens_after)
    lin = d.model.linear_bytes(bsz)
    step_bytes = d.step_bytes(lens_before, lens_after)
    dominant = max(kdur, key=lambda k: kdur[k] * per_step[k])
    counters = committed_figures(GEMM_COUNTER_PROFILE, "gemm-counters")
    if bsz == 32 and args.model == "llama3-8b":
        for k in kernels:
            if k in counters:
                kernels[k]["counters"] = counters[k]
    layer_linear_b = sum(lin[k] for k in ("qkv", "o", "gate_up", "down"))
    layer_linear_s = sum(kdur[k] for k in (("qkv", "o", "mlp") if "mlp" in kdur else ("qkv", "o", "gate_up", "down")))
    achieved = per_launch[dominant] / kdur[dominant] / 1e9
    traffic = None
    if dominant == "attn" and args.model == "llama3-8b" and bsz == 32 and d.n_layers == s.layers:
        t = committed_figures(ATTN_TRAFFIC_PROFILE, "bench-traffic").get("attn")
        traffic = (int(t["bytes_per_launch"]), int(t["algorithmic_bytes"])) if t else None
    out = {
        "metric": METRIC, "value": round(bsz / (ms * 1e-3), 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": DTYPE, "data": DATA,
        "config": {
            "workload": f"{args.model}-shaped int8 decode step (int8 linears + paged-attn decode), batch {bsz}",
            "batch": bsz, "layers": d.n_layers, "hidden": s.hidden, "heads": s.heads, "kv_heads": s.kv_heads,
            "head_dim": s.head_dim, "intermediate": s.intermediate, "vocab": s.vocab,
            "contexts": f"U[{args.ctx_lo},{args.ctx_hi}] seed 0", "block_size": d.bs,
            "pool_blocks": args.pool_blocks, "hip_graph": not args.no_graph, "fused_mlp": "mlp" in kdur,
            "parallelism": "none (1 GPU)",
        },
        "step_hbm_bytes": step_bytes,
        "step_gbps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "step_hbm_frac": frac(step_bytes / (ms * 1e-3) / 1e9),
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": frac(achieved), "traffic": traffic[0] if traffic else None,
                     "traffic_note": (f"HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE "
                                      f"(copy-calibrated), profiles/{os.path.basename(ATTN_TRAFFIC_PROFILE)}; "
                                      f"{traffic[1]} algorithmic bytes at that run's contexts") if traffic else None},
        "kernels": kernels,
        "layer_linears": {"avg_us": round(layer_linear_s * 1e6, 2), "bytes": layer_linear_b,
                          "gbps": round(layer_linear_b / layer_linear_s / 1e9, 1),
                          "frac": frac(layer_linear_b / layer_linear_s / 1e9)},
        "hbm_copy": copy_bandwidth(),
        "setup_s": round(d.setup_s, 1),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_step_baseline(s, bsz, d.lens.tolist(), d.n_layers)
    return out


# ---------------------------------------------------------------------------------------------
# Config 2: paged decode attention alone, and the gather ceiling
# ---------------------------------------------------------------------------------------------
def config2_attention(args, pool, layers: int) -> dict:
    """torch.manual_seed(0); seq_lens ~ U{128..4096} for 32 rows; each row takes ceil(S/16) ids
    from one randperm(16384); q [32, 32, 1, 128] N(0, 1) fp16, K/V N(0, 1) (the pool's random
    contents); scale 1/sqrt(128). Timed over ``layers`` layer views of the pool (one call per
    layer, as in the step) so no call re-reads K/V from the MALL."""
    import torch

    from oracle.paged_attention import decode_rows_fp32
    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.paged_attention_hip import _decode
    from runtime_amd.phase2.roofline import attention_hbm_bytes

    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, bs = 32, 32, 8, 128, 16
    nb = pool.shape.num_blocks
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
    qd, td, ld = q.to(dev), tables.to(dev), lens.to(device=dev, dtype=torch.int32)
    scale = D**-0.5

    def run():
        for li in range(layers):
            _decode(qd, pool.k_layer_view(li), pool.v_layer_view(li), td, ld, scale, Hq // Hkv)
    t = graph_time(run, layers, reps=max(2, args.kernel_steps))
    byts = attention_hbm_bytes(lens.tolist(), Hkv, D, Hq, bs)
    kv_bytes = int(lens.sum()) * Hkv * D * 2 * 2
    lib = _hip.load()
    sink = torch.zeros(2, dtype=torch.int32, device=dev)
    ceiling = {}
    for mode, name in ((0, "decode_pattern"), (1, "whole_blocks")):
        def probe(mode=mode):
            for li in range(layers):
                k, v = pool.k_layer_view(li), pool.v_layer_view(li)
                _hip.check(lib.mx_kv_gather_probe(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), td.data_ptr(),
                                                  td.stride(0), td.shape[1], ld.data_ptr(), B, Hkv, D, bs, nb, mode,
                                                  sink.data_ptr(), _hip.stream_handle(dev)), "mx_kv_gather_probe")
        tp = graph_time(probe, layers, reps=max(2, args.kernel_steps))
        ceiling[name] = {"avg_us": round(tp * 1e6, 2), "gbps": round(kv_bytes / tp / 1e9, 1),
                         "frac": frac(kv_bytes / tp / 1e9)}
    achieved = byts / t / 1e9
    out = {
        "workload": "paged decode attention, B 32, Hq 32, Hkv 8, D 128, block 16, contexts U[128,4096] "
                    "(torch.manual_seed(0)), pool 16384 blocks x 32 layers",
        "avg_us": round(t * 1e6, 2), "bytes_per_call": byts, "gbps": round(achieved, 1), "frac": frac(achieved),
        "gather_ceiling": dict(ceiling, what="the same K/V reads without the math (mx_kv_gather_probe), "
                                              f"{kv_bytes} K/V bytes per call"),
        "kv_frac_of_gather_ceiling": round(ceiling["decode_pattern"]["avg_us"] / (t * 1e6), 4),
    }
    if not args.no_cpu_baseline:
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        ids = torch.unique(tables[tables >= 0])
        kc = pool.k_layer_view(0)[ids.to(dev)].cpu()
        vc = pool.v_layer_view(0)[ids.to(dev)].cpu()
        remap = torch.full((nb,), -1, dtype=torch.int32)
        remap[ids] = torch.arange(ids.numel(), dtype=torch.int32)
        tc = remap[tables.long()]
        lens_l = lens.tolist()
        decode_rows_fp32(q, kc, vc, tc, lens_l, scale, Hq // Hkv)  # warm
        t_cpu, reps = repeat_for(lambda: decode_rows_fp32(q, kc, vc, tc, lens_l, scale, Hq // Hkv), CPU_SAMPLE_S)
        out["cpu_baseline"] = {"value": round(byts / t_cpu / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
                               "sample": "the per-row fp32 oracle (oracle.paged_attention.decode_rows_fp32) on "
                                         f"the same inputs, x{reps}", "ms_per_call": round(t_cpu * 1e3, 1),
                               "sample_seconds": round(t_cpu * reps, 2)}
    return out


# ---------------------------------------------------------------------------------------------
# Configs 1 and 4: the int8 linears alone
# ---------------------------------------------------------------------------------------------
def config14_linears(args) -> tuple[dict, dict]:
    """Config 1 (x [1, 4096] @ W [4096, 4096], seed 0) and config 4 (the Llama-3-8B projections,
    seed 1000 + shape index, M in {1, 8, 32, 64}) through ``int8_linear``. Weights are N(0, 0.02)
    quantized on the device; each timed graph walks over enough distinct weight copies
    (> 512 MB) that no launch reads its weights from the 256 MB MALL. The CPU oracle (fp32 x @
    dequantized W^T) is timed per shape and M."""
    import numpy as np
    import torch

    from oracle import int8_quant
    from runtime_amd.phase2.int8_linear import int8_linear, pack_weight, quantize_weight
    from runtime_amd.phase2.roofline import linear_hbm_bytes

    dev = torch.device("cuda:0")
    shapes = [("config1", 4096, 4096, [1])] + [(n, k, nn, [1, 8, 32, 64]) for n, k, nn in
                                               (("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 28672),
                                                ("down", 14336, 4096))]
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    counters = committed_figures(SWEEP_COUNTER_PROFILE, "gemm-counters")
    rows = []
    for idx, (name, k, n, ms) in enumerate(shapes):
        g = torch.Generator(device=dev).manual_seed(0 if name == "config1" else 1000 + idx - 1)
        copies = max(4, math.ceil(600e6 / (n * k)))
        weights = []
        for _ in range(copies):
            q, sc = quantize_weight(torch.randn(n, k, generator=g, device=dev) * 0.02)
            weights.append((pack_weight(q), sc))
        w_cpu = None
        if not args.no_cpu_baseline:
            # The oracle's operand: int8 values of the same shape (drawn on the host; a timing
            # baseline needs the shape, not these particular values) dequantized once with the
            # device's scales.
            q_rows = np.random.default_rng(idx).integers(-127, 128, size=(n, k), dtype=np.int8)
            w_cpu = torch.from_numpy(int8_quant.dequantize(q_rows, weights[0][1].cpu().numpy()))
        for m in ms:
            x = torch.randn(m, k, generator=g, device=dev).half()
            y = torch.empty(m, n, dtype=torch.float16, device=dev)

            def run():
                for packed, sc in weights:
                    int8_linear(x, packed, sc, None, n, out=y)
            t = graph_time(run, copies)
            byts = linear_hbm_bytes(m, n, k)
            gbps = byts / t / 1e9
            row = {"shape": name, "m": m, "n": n, "k": k, "avg_us": round(t * 1e6, 2), "bytes": byts,
                   "gbps": round(gbps, 1), "frac": frac(gbps)}
            key = f"{name}_m{m}"
            if key in counters:
                row["counters"] = counters[key]
            if w_cpu is not None:
                xf = x.float().cpu()
                xf @ w_cpu.T
                t_cpu, reps = repeat_for(lambda: xf @ w_cpu.T, CPU_SAMPLE_S / 20)
                row["cpu_baseline"] = {"us": round(t_cpu * 1e6, 1), "gbps": round(byts / t_cpu / 1e9, 2),
                                       "calls": reps}
            rows.append(row)
        del weights, w_cpu
        torch.cuda.empty_cache()
    c1 = rows[0]
    cpu_note = {"unit": "GB/s", "cores": cores, "kind": "port",
                "sample": "the CPU oracle per shape and M: fp32 x @ W^T on weights dequantized once "
                          "(oracle.int8_quant.dequantize), mean over 0.5 s of calls after one warm-up"}
    config1 = {
        "workload": "int8 linear x [1,4096] @ W [4096,4096] (seed 0)",
        "avg_us": c1["avg_us"], "bytes_per_call": c1["bytes"], "gbps": c1["gbps"], "frac": c1["frac"],
    }
    if "counters" in c1:
        config1["counters"] = dict(c1["counters"], profile=os.path.relpath(SWEEP_COUNTER_PROFILE, HERE))
    if "cpu_baseline" in c1:
        config1["cpu_baseline"] = dict(cpu_note, value=c1["cpu_baseline"]["gbps"], us_per_call=c1["cpu_baseline"]["us"])
    sweep_rows = rows[1:]
    config4 = {
        "workload": "Llama-3-8B int8 projections qkv 4096->6144, o 4096->4096, gate_up 4096->28672, "
                    "down 14336->4096 at M in {1,8,32,64}; each launch alone (split-K shapes include their "
                    "reduce launch)",
        "rows": sweep_rows,
        "per_layer": {f"m{m}": {"avg_us": round(sum(r["avg_us"] for r in sweep_rows if r["m"] == m), 2),
                                "bytes": sum(r["bytes"] for r in sweep_rows if r["m"] == m),
                                "frac": frac(sum(r["bytes"] for r in sweep_rows if r["m"] == m)
                                             / (sum(r["avg_us"] for r in sweep_rows if r["m"] == m) * 1e-6) / 1e9)}
                      for m in (1, 8, 32, 64)},
    }
    if not args.no_cpu_baseline:
        config4["cpu_baseline"] = cpu_note
    return config1, config4


# ---------------------------------------------------------------------------------------------
# Calibration probes: what one CU streams, and what a launch costs inside a graph
# ---------------------------------------------------------------------------------------------
STREAM_PROBE_SHAPES = ((1, 64 << 10), (1, 1 << 20), (32, 256 << 10), (256, 64 << 10), (256, 256 << 10),
                       (512, 256 << 10), (512, 1 << 20))
LAUNCH_PROBE_SHAPES = ((0, 256), (16 * 256, 256), (4 << 20, 256), (16 << 20, 256), (64 << 20, 1024))


def calibration_probes(args) -> dict:
    """The tables the kernels' shapes were chosen from, measured on this GPU.

    * stream: G workgroups of T threads each read their own contiguous run of B bytes
      (``mx_stream_probe``: non-temporal 16-byte loads, 4 in flight per thread), 20 launches per graph
      at distinct offsets of a 2 GiB buffer (a run is not re-read until 2 GiB later, past the 256 MB
      MALL); per launch us and GB/s.
    * launch: a graph of 100 launches of ``mx_launch_probe`` that do nothing or write the given bytes
      (equal shares per workgroup); per launch us.
    """
    import torch

    from runtime_amd.phase2 import _hip

    lib = _hip.load()
    dev = torch.device("cuda:0")
    span_total = 2 << 30
    buf = torch.empty(span_total, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    launches = 20
    stream = []
    for wgs, per in STREAM_PROBE_SHAPES:
        span = wgs * per
        n_off = max(1, min(launches, span_total // span))
        for threads in (256, 512, 1024):
            def run(wgs=wgs, per=per, span=span, n_off=n_off, threads=threads):
                st = _hip.stream_handle(dev)
                for i in range(launches):
                    _hip.check(lib.mx_stream_probe(buf.data_ptr(), span_total, (i % n_off) * span, per, wgs, threads,
                                                   sink.data_ptr(), st), "mx_stream_probe")
            t = graph_time(run, launches)
            stream.append({"workgroups": wgs, "bytes_per_workgroup": per, "threads": threads,
                           "us": round(t * 1e6, 2), "gbps": round(span / t / 1e9, 1)})
    del buf
    torch.cuda.empty_cache()
    print("[probes] stream done", file=sys.stderr, flush=True)
    dst = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    launch = []
    for nbytes, wgs in LAUNCH_PROBE_SHAPES:
        def run(nbytes=nbytes, wgs=wgs):
            st = _hip.stream_handle(dev)
            for _ in range(100):
                _hip.check(lib.mx_launch_probe(dst.data_ptr(), dst.numel(), nbytes, wgs, st), "mx_launch_probe")
        t = graph_time(run, 100)
        launch.append({"bytes_written": nbytes, "workgroups": wgs, "us": round(t * 1e6, 2)})
    del dst
    torch.cuda.empty_cache()
    print("[probes] launch done", file=sys.stderr, flush=True)
    handoff, barrier, chain = handoff_probes()
    gather = gather_sweep(args)
    print("[probes] gather done", file=sys.stderr, flush=True)
    return {"stream": stream, "launch": launch, "handoff": handoff, "barrier": barrier, "chain": chain,
            "gather": gather,
            "what": "mx_stream_probe (per-workgroup contiguous runs, 20 launches per graph over 2 GiB), "
                    "mx_launch_probe (graphs of 100 launches), mx_handoff_probe (graphs of 20 calls), "
                    "mx_barrier_probe (per barrier: a 200-round launch less a 0-round one), mx_chain_probe "
                    "(per phase, graph of one launch per phase vs one persistent launch), "
                    "mx_run_gather_probe / mx_kv_gather_probe over config 2's K/V runs (one call per layer of "
                    "a 32-layer pool)"}


HANDOFF_SHAPES = ((256, 4), (512, 16), (1024, 4), (2048, 8))
HANDOFF_MODES = ("partials alone", "+ a reduce launch", "last arriver, agent-scope release/acquire",
                 "last arriver, seq_cst fences", "last arriver, write-through stores + ticket, no fences")
BARRIER_MODES = ("one device-scope counter, thread 0 polls", "one flag per workgroup, one wave polls all",
                 "8 group counters, every workgroup polls all 8",
                 "8 group counters + 1 KiB per workgroup handed over through device-coherent stores and loads",
                 "8 group counters + the same 1 KiB behind agent-scope release/acquire fences")
CHAIN_PER_WG = (8 << 10, 32 << 10, 64 << 10, 128 << 10, 256 << 10)


def handoff_probes():
    """What handing data between the workgroups of one launch costs against a launch boundary.

    * handoff: groups of G workgroups each write an 8 KiB fp32 partial that one workgroup (or a second
      launch) must sum (``mx_handoff_probe``, five ways); per call us, graphs of 20 calls.
    * barrier: 256 resident workgroups of 512 threads pass grid barriers of five kinds
      (``mx_barrier_probe``); us per barrier = (200-round launch - 0-round launch) / 200.
    * chain: phases that each stream distinct weight bytes (256 workgroups x B bytes) and hand 1 KiB per
      workgroup to the next phase, as a graph of one launch per phase or as one persistent launch that
      issues each phase's first loads before its barrier (``mx_chain_probe``); us per phase, enough
      phases to read at least 512 MB (past the 256 MB MALL).
    Every call's error word (time-outs, wrong hand-off values) and result are checked.
    """
    import torch

    from runtime_amd.phase2 import _hip

    lib = _hip.load()
    dev = torch.device("cuda:0")
    handoff = []
    for wgs, g in HANDOFF_SHAPES:
        part = torch.empty(wgs * 2048, dtype=torch.float32, device=dev)
        out = torch.empty(wgs // g * 2048, dtype=torch.float32, device=dev)
        tickets = torch.zeros(wgs // g, dtype=torch.int32, device=dev)
        row = {"workgroups": wgs, "group": g}
        for mode, name in enumerate(HANDOFF_MODES):
            def run(mode=mode):
                st = _hip.stream_handle(dev)
                for _ in range(20):
                    _hip.check(lib.mx_handoff_probe(part.data_ptr(), part.numel() * 4, out.data_ptr(), out.numel() * 4,
                                                    tickets.data_ptr(), tickets.numel() * 4, wgs, g, mode, st),
                               "mx_handoff_probe")
            row[name] = round(graph_time(run, 20) * 1e6, 2)
        if int(tickets.abs().sum()) != 0:
            raise RuntimeError("mx_handoff_probe left a ticket set")
        handoff.append(row)
        del part, out, tickets
    print("[probes] handoff done", file=sys.stderr, flush=True)
    n = 256
    sync = torch.zeros(16 + n, dtype=torch.int32, device=dev)
    hand = torch.zeros(2 * n * 256, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    barrier = []
    for mode, name in enumerate(BARRIER_MODES):
        t = {}
        for rounds in (0, 200):
            def run(rounds=rounds, mode=mode):
                _hip.check(lib.mx_barrier_probe(sync.data_ptr(), sync.numel() * 4, hand.data_ptr(), hand.numel() * 4, n,
                                                rounds, mode, err.data_ptr(), _hip.stream_handle(dev)),
                           "mx_barrier_probe")
            t[rounds] = graph_time(run, 1, reps=10)
        if int(err) != 0:
            raise RuntimeError(f"mx_barrier_probe mode {mode}: error word {int(err)}")
        barrier.append({"barrier": name, "workgroups": n, "us_per_barrier": round((t[200] - t[0]) / 200 * 1e6, 2)})
    print("[probes] barrier done", file=sys.stderr, flush=True)
    chain = []
    span = max(per * n * max(8, -(-(512 << 20) // (per * n))) for per in CHAIN_PER_WG)
    src = torch.empty(span, dtype=torch.uint8, device=dev)
    src.fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for per in CHAIN_PER_WG:
        phases = min(256, max(8, -(-(512 << 20) // (per * n))))
        row = {"weight_bytes_per_phase": per * n, "phases": phases}
        for persistent, name in ((0, "graph of kernels"), (1, "persistent kernel")):
            def run(persistent=persistent, per=per, phases=phases):
                st = _hip.stream_handle(dev)
                calls = [(0, phases)] if persistent else [(p, 1) for p in range(phases)]
                for p0, count in calls:
                    _hip.check(lib.mx_chain_probe(src.data_ptr(), span, per, n, p0, count, persistent, sync.data_ptr(),
                                                  sync.numel() * 4, hand.data_ptr(), hand.numel() * 4, err.data_ptr(),
                                                  sink.data_ptr(), st), "mx_chain_probe")
            row[name] = round(graph_time(run, phases) * 1e6, 2)
            if int(err) != 0:
                raise RuntimeError(f"mx_chain_probe ({name}, {per} bytes per workgroup): error word {int(err)}")
        chain.append(row)
        print(f"[probes] chain {per} bytes per workgroup done", file=sys.stderr, flush=True)
    del src
    torch.cuda.empty_cache()
    return handoff, barrier, chain


# (waves, runs in flight, streaming, load pattern: 0 1 KiB contiguous, 1/2 the attention kernel's operand loads)
GATHER_SWEEP = ((1024, 2, 1, 0), (1024, 3, 1, 0), (2048, 1, 1, 0), (2048, 2, 1, 0), (2048, 3, 1, 0), (4096, 2, 1, 0),
                (4096, 4, 1, 0), (2048, 2, 0, 0), (1024, 3, 0, 0), (2048, 2, 1, 1), (2048, 2, 1, 2), (1024, 2, 1, 2),
                (2048, 2, 1, 3), (1024, 2, 1, 3), (2048, 2, 1, 4), (1024, 2, 1, 4))


def gather_sweep(args) -> dict:
    """Config 2's K/V reads (torch.manual_seed(0) contexts and tables, the bench's interleaved 16384-block
    pool of 32 layers) without the math: each (block, kv-head)'s K and V runs are one 8 KiB run of the
    pool. W waves take equal shares of a layer's runs, R runs in flight per wave, streaming or default
    loads (``mx_run_gather_probe``), one call per layer; beside it the attention kernel's own partition
    and loads (``mx_kv_gather_probe`` mode 0) and whole-block workgroups (mode 1)."""
    import torch

    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool

    lib = _hip.load()
    dev = torch.device("cuda:0")
    B, Hkv, D, bs, nb, layers = 32, 8, 128, 16, 16384, 32
    pool = GpuKVBlockPool(num_blocks=nb, block_size_tokens=bs, num_layers=layers, num_kv_heads=Hkv, head_dim=D,
                          dtype=torch.float16, device=dev)
    pool._ensure_pools()
    k0 = pool.k_layer_view(0)
    if pool.v_layer_view(0).data_ptr() - k0.data_ptr() != bs * D * 2:
        raise RuntimeError("the gather sweep needs the interleaved pool (K and V runs of a block adjacent)")
    torch.manual_seed(0)
    lens = torch.randint(128, 4097, (B,))
    perm = torch.randperm(nb)
    nblk = [math.ceil(int(x) / bs) for x in lens]
    tables = torch.zeros(B, max(nblk), dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        tables[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    ids = torch.cat([tables[b, :n] for b, n in enumerate(nblk)]).long()  # row-major, as the segments run
    base = pool._k_pool.data_ptr()
    base_bytes = pool._k_pool.untyped_storage().nbytes()  # the whole pool (K and V of every layer)
    sblk, shead = k0.stride(0) * 2, k0.stride(1) * 2
    offs = []
    for li in range(layers):
        lo = pool.k_layer_view(li).data_ptr() - base
        heads = torch.arange(Hkv, dtype=torch.long) * shead
        offs.append((lo + ids[:, None] * sblk + heads[None, :]).flatten().to(dev))
    n_runs = int(offs[0].numel())
    run_bytes = 2 * bs * D * 2
    sink = torch.zeros(2, dtype=torch.int32, device=dev)
    kv_bytes = n_runs * run_bytes
    rows = []
    for waves, r, streaming, pattern in GATHER_SWEEP:
        def run(waves=waves, r=r, streaming=streaming, pattern=pattern):
            st = _hip.stream_handle(dev)
            for li in range(layers):
                _hip.check(lib.mx_run_gather_probe(base, base_bytes, offs[li].data_ptr(), n_runs, run_bytes, waves, r,
                                                   streaming, pattern, sink.data_ptr(), st), "mx_run_gather_probe")
        t = graph_time(run, layers, reps=max(2, args.kernel_steps))
        rows.append({"waves": waves, "runs_in_flight": r, "loads": "streaming" if streaming else "default",
                     "pattern": ("1 KiB contiguous", "attention operands, streaming",
                                 "attention operands, K first halves default",
                                 "attention operands, K staged through LDS in whole rows",
                                 "K staged through LDS, rows permuted so V loads are 1 KiB contiguous")[pattern],
                     "us": round(t * 1e6, 2), "gbps": round(kv_bytes / t / 1e9, 1), "frac": frac(kv_bytes / t / 1e9)})
    td, ld = tables.to(dev), lens.to(device=dev, dtype=torch.int32)
    kernel = {}
    for mode, name in ((0, "attention_partition"), (1, "whole_blocks")):
        def probe(mode=mode):
            for li in range(layers):
                k, v = pool.k_layer_view(li), pool.v_layer_view(li)
                _hip.check(lib.mx_kv_gather_probe(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), td.data_ptr(),
                                                  td.stride(0), td.shape[1], ld.data_ptr(), B, Hkv, D, bs, nb, mode,
                                                  sink.data_ptr(), _hip.stream_handle(dev)), "mx_kv_gather_probe")
        t = graph_time(probe, layers, reps=max(2, args.kernel_steps))
        kernel[name] = {"us": round(t * 1e6, 2), "gbps": round(kv_bytes / t / 1e9, 1), "frac": frac(kv_bytes / t / 1e9)}
    del pool
    torch.cuda.empty_cache()
    return {"runs_per_call": n_runs, "run_bytes": run_bytes, "kv_bytes_per_call": kv_bytes, "sweep": rows,
            "kv_gather_probe": kernel}


# ---------------------------------------------------------------------------------------------
# Config 3: the Qwen2-0.5B-shaped step
# ---------------------------------------------------------------------------------------------
def config3_qwen(args) -> dict:
    import torch

    from runtime_amd.phase2.decode_step import QWEN2_05B

    steps = args.steps
    d = Decoder(QWEN2_05B, batch=16, lo=512, hi=2048, pool_blocks=4096,
                headroom=args.warmup + 1 + GRAPH_WARMUP + steps + 2)
    lens_before = d.seq_lens.cpu().tolist()
    ms = time_step(d.step, steps, args.warmup)
    lens_after = d.seq_lens.cpu().tolist()
    byts = d.step_bytes(lens_before, lens_after)
    gbps = byts / (ms * 1e-3) / 1e9
    kdur, _, per_step, kernels = family_table(d, args, lens_after)
    out = {
        "workload": "Qwen2-0.5B-shaped int8 decode step (hidden 896, 24 layers, 14/2 heads, head_dim 64, "
                    "SwiGLU 4864, vocab 151936, qkv bias), batch 16, contexts U[512,2048] seed 0, block 16, "
                    "HIP graph",
        "value": round(16 / (ms * 1e-3), 2), "unit": "tokens/s", "ms_per_step": round(ms, 4),
        "step_hbm_bytes": byts, "gbps": round(gbps, 1), "frac": frac(gbps),
        "roofline_tokens_per_s": round(16 / (byts / (HBM_PEAK_GBPS * 1e9)), 1),
        "kernels": kernels,
        # Step time not covered by the families' own graph-replay time: the RMSNorm/residual
        # launches, the embedding and argmax, and the dependency gaps between launches.
        "other_us_per_step": round(ms * 1e3 - sum(kdur[k] * per_step[k] for k in kdur) * 1e6, 1),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_step_baseline(QWEN2_05B, 16, d.lens.tolist(), d.n_layers)
    del d
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------------------------
# Config 5: shared-prefix continuous batching on the headline model
# ---------------------------------------------------------------------------------------------
def config5_prefix(args, model, bsz: int = 128) -> dict:
    """``bsz`` rows in 16 groups whose rows alias one 1024-token prefix (block ids shared, stored
    once), contexts U[1, 8192]. Every 16 steps the rows b with b % 8 == epoch % 8 finish and new
    requests of the same group join their slots (freed blocks reused; tables, lengths and tokens
    rewritten in place between replays of one captured step graph, inside the timed region).
    ``value`` is tokens/s; the HBM figure counts weights + unique K/V bytes."""
    import torch

    from runtime_amd.phase2.paged_attention_hip import _decode
    from runtime_amd.phase2.paged_kv_kernel import GpuKVBlockPool
    from runtime_amd.phase2.prefix_batch import PrefixBatch

    dev = torch.device("cuda:0")
    shape, n_layers = model.shape, len(model.layers)
    bs, lo, hi, steps = 16, 1, 8192, args.prefix_steps
    total_steps = args.warmup + 1 + GRAPH_WARMUP + steps
    num_blocks = 40960
    t_setup = time.perf_counter()
    pb = PrefixBatch(batch=bsz, groups=PREFIX_GROUPS, prefix_tokens=PREFIX_TOKENS, lo=lo, hi=hi, block_size=bs,
                     num_blocks=num_blocks, headroom=total_steps + ROTATE_EVERY, seed=0)
    shared_before = model.shared_kv_blocks
    model.shared_kv_blocks = not args.stream_shared_kv
    pool = GpuKVBlockPool(num_blocks=num_blocks, block_size_tokens=bs, num_layers=n_layers,
                          num_kv_heads=shape.kv_heads, head_dim=shape.head_dim, dtype=torch.float16, device=dev,
                          kv_layout=args.kv_layout)
    pool._ensure_pools()
    gk = torch.Generator(device=dev).manual_seed(1)
    fill_normal(pool._k_pool, gk)
    fill_normal(pool._v_pool, gk)
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
    for _ in range(GRAPH_WARMUP):
        graph.replay()
        pb.advance(1)
    torch.cuda.synchronize()
    assert seq_lens.cpu().tolist() == pb.lens.tolist(), "device lengths diverged from the schedule"

    kv_token_bytes = n_layers * shape.kv_heads * shape.head_dim * 2 * 2

    def rotation(k: int) -> list[int]:
        if k == 0 or k % ROTATE_EVERY:
            return []
        return [b for b in range(bsz) if b % 8 == (k // ROTATE_EVERY) % 8]

    rotated = 0
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for k in range(steps):
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
    ms = start.elapsed_time(end) / steps
    assert seq_lens.cpu().tolist() == pb.lens.tolist(), "device lengths diverged from the schedule"

    # Byte accounting, outside the timed region: the same seeded schedule replayed on the host.
    acct = PrefixBatch(batch=bsz, groups=PREFIX_GROUPS, prefix_tokens=PREFIX_TOKENS, lo=lo, hi=hi, block_size=bs,
                       num_blocks=num_blocks, headroom=total_steps + ROTATE_EVERY, seed=0)
    acct.advance(args.warmup + 1 + GRAPH_WARMUP)
    uniq, logical = [], []
    for k in range(steps):
        rows = rotation(k)
        if rows:
            acct.rotate(rows)
        uniq.append(acct.unique_tokens(1))
        logical.append(acct.logical_tokens(1))
        acct.advance(1)
    assert acct.lens.tolist() == pb.lens.tolist()

    # Attention family at the final state (one call per layer, one graph).
    q = torch.randn(bsz, shape.heads, 1, shape.head_dim, generator=gk, device=dev).half()
    lens_attn = (seq_lens + 1).to(torch.int32)

    def attn():
        for li in range(n_layers):
            _decode(q, pool.k_layer_view(li), pool.v_layer_view(li), tables_d, lens_attn, shape.head_dim**-0.5,
                    shape.group, shared_blocks=model.shared_kv_blocks)
    attn_s = graph_time(attn, n_layers, args.kernel_steps)
    final_uniq = pb.unique_tokens(1) * shape.kv_heads * shape.head_dim * 2 * 2
    final_logical = pb.logical_tokens(1) * shape.kv_heads * shape.head_dim * 2 * 2
    lin = model.linear_bytes(bsz)
    weight_bytes = n_layers * (lin["qkv"] + lin["o"] + lin["gate_up"] + lin["down"]) + lin["lm_head"]
    uniq_b = sum(uniq) / len(uniq) * kv_token_bytes
    logical_b = sum(logical) / len(logical) * kv_token_bytes
    model.shared_kv_blocks = shared_before
    del pool, graph
    torch.cuda.empty_cache()
    gbps = (weight_bytes + uniq_b) / (ms * 1e-3) / 1e9
    return {
        "workload": f"llama3-8b-shaped int8 decode step, {bsz} rows in {PREFIX_GROUPS} groups sharing a "
                    f"{PREFIX_TOKENS}-token prefix (aliased blocks), contexts U[{lo},{hi}], {bsz // 8} rows finish "
                    f"and join every {ROTATE_EVERY} steps, HIP graph",
        "value": round(bsz / (ms * 1e-3), 2), "unit": "tokens/s", "steps": steps, "ms_per_step": round(ms, 4),
        "rows_rotated": rotated, "kv_logical_bytes_per_step": int(logical_b),
        "kv_unique_bytes_per_step": int(uniq_b), "weight_bytes_per_step": weight_bytes,
        "gbps_unique": round(gbps, 1), "frac_unique": frac(gbps),
        "attn": {"avg_us": round(attn_s * 1e6, 2), "unique_bytes": final_uniq, "logical_bytes": final_logical,
                 "gbps_unique": round(final_uniq / attn_s / 1e9, 1),
                 "gbps_logical": round(final_logical / attn_s / 1e9, 1)},
        "setup_s": round(setup_s, 1),
        "cpu_baseline": None, "cpu_baseline_note": "not CPU-timed (68 GB of logical K/V per step); the "
                                                   "configuration asks for none",
    }


# ---------------------------------------------------------------------------------------------
# Counter-pass probes
# ---------------------------------------------------------------------------------------------
def traffic_probe(args) -> int:
    """Kernels for one rocprofv3 --pmc pass, nothing else: REPS rounds of one kernel family's
    launches of the headline step (attention: one call per layer, so no launch re-reads the
    previous one's K/V from the 256 MB MALL; linears: the four projections of every layer, as
    the step launches them), then one copy of COPY_PROBE_BYTES, whose counter reading
    calibrates FETCH_SIZE / WRITE_SIZE (it reads and writes exactly that many bytes)."""
    import torch

    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.decode_step import LLAMA3_8B, QWEN2_05B
    from runtime_amd.phase2.roofline import attention_hbm_bytes

    _hip.load()
    if args.probe_family == "sweep":
        return sweep_probe(args)
    shape = LLAMA3_8B if args.model == "llama3-8b" else QWEN2_05B
    headroom = args.warmup + args.steps + args.kernel_steps + 2  # the bench's table width
    d = Decoder(shape, args.batch, args.ctx_lo, args.ctx_hi, args.pool_blocks, headroom, layers=args.layers,
                kv_layout=args.kv_layout)
    fams = family_launches(d)
    names = ["attn"] if args.probe_family == "attn" else ["qkv", "o", "gate_up", "down"]
    for name in names:
        fams[name][0]()  # eager warm-up: workspaces
    torch.cuda.synchronize()
    for _ in range(args.traffic_probe):
        for name in names:
            fams[name][0]()
    src = torch.empty(COPY_PROBE_BYTES // 2, dtype=torch.float16, device=d.dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    lin = d.model.linear_bytes(d.batch)
    per_launch = {"attn": attention_hbm_bytes([x + 1 for x in d.lens.tolist()], shape.kv_heads, shape.head_dim,
                                              shape.heads, d.bs), **lin}
    print(json.dumps({"probe": args.probe_family, "launches_per_family": args.traffic_probe * d.n_layers + d.n_layers,
                      "bytes_per_launch": {n: per_launch[n] for n in names}, "copy_bytes": COPY_PROBE_BYTES}),
          flush=True)
    return 0


def sweep_probe(args) -> int:
    """Counter-pass probe of configs 1 and 4: ``int8_linear`` alone at M = ``--batch`` on each
    Llama-3-8B projection (and config 1's 4096x4096 at M = 1), as ``config14_linears`` times it:
    one warm-up round and REPS rounds over enough distinct weight copies (> 600 MB) that no launch
    finds its weights in the 256 MB MALL, shape after shape, then the 1 GiB calibration copy. Every
    call is one GEMV/GEMM dispatch, followed by a ``reduce_kernel`` dispatch where K is split; the
    printed manifest gives the calls per shape in dispatch order."""
    import torch

    from runtime_amd.phase2.int8_linear import int8_linear, linear_splits, pack_weight, quantize_weight
    from runtime_amd.phase2.roofline import linear_hbm_bytes

    dev, m = torch.device("cuda:0"), args.batch
    shapes = ([("config1", 4096, 4096)] if m == 1 else []) + [("qkv", 4096, 6144), ("o", 4096, 4096),
                                                             ("gate_up", 4096, 28672), ("down", 14336, 4096)]
    cases = []
    seeds = {"config1": 0, "qkv": 1000, "o": 1001, "gate_up": 1002, "down": 1003}  # config14_linears' seeds
    for name, k, n in shapes:
        g = torch.Generator(device=dev).manual_seed(seeds[name])
        copies = max(4, math.ceil(600e6 / (n * k)))
        weights = []
        for _ in range(copies):
            q, sc = quantize_weight(torch.randn(n, k, generator=g, device=dev) * 0.02)
            weights.append((pack_weight(q), sc))
        x = torch.randn(m, k, generator=g, device=dev).half()
        y = torch.empty(m, n, dtype=torch.float16, device=dev)
        cases.append((name, n, k, weights, x, y))
    torch.cuda.synchronize()
    manifest = []
    for name, n, k, weights, x, y in cases:
        for _ in range(1 + args.traffic_probe):
            for packed, sc in weights:
                int8_linear(x, packed, sc, None, n, out=y)
        manifest.append({"shape": name, "m": m, "n": n, "k": k, "calls": (1 + args.traffic_probe) * len(weights),
                         "splits": linear_splits(m, n, k), "bytes_per_call": linear_hbm_bytes(m, n, k)})
    src = torch.empty(COPY_PROBE_BYTES // 2, dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "sweep", "m": m, "manifest": manifest, "copy_bytes": COPY_PROBE_BYTES}), flush=True)
    return 0


# ---------------------------------------------------------------------------------------------
def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards without exchange; see the design notes). Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    from runtime_amd.phase2 import _hip
    from runtime_amd.phase2.decode_step import LLAMA3_8B, QWEN2_05B

    _hip.load()
    torch.cuda.set_device(0)
    if args.traffic_probe:
        return traffic_probe(args)
    t_start = time.perf_counter()

    def done(name):
        print(f"[bench] {name} done at {time.perf_counter() - t_start:.1f} s", file=sys.stderr, flush=True)

    if args.workload == "linear-sweep":
        c1, c4 = config14_linears(args)
        print(json.dumps({"metric": "int8 linear algorithmic HBM GB/s (config 1; config 4 in 'config4')",
                          "value": c1["gbps"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
                          "dtype": DTYPE, "data": DATA, "config": {"workload": c1["workload"]},
                          "config1": c1, "config4": c4}), flush=True)
        return 0
    if args.workload == "probes":
        pr = calibration_probes(args)
        print(json.dumps({"metric": "calibration probes (per-CU streaming, launch floor in a HIP graph, in-launch "
                                    "hand-offs, K/V gather)", "n_gpus": 1, "data": DATA, **pr}), flush=True)
        return 0
    if args.workload == "qwen":
        c3 = config3_qwen(args)
        print(json.dumps(dict(metric=METRIC, n_gpus=1, dtype=DTYPE, data=DATA, higher_is_better=True,
                              config={"workload": c3["workload"]}, **c3)), flush=True)
        return 0
    shape = LLAMA3_8B if args.model == "llama3-8b" else QWEN2_05B
    if args.workload == "prefix-batch":
        from runtime_amd.phase2.decode_step import Int8DecodeModel

        model = Int8DecodeModel(shape, device="cuda:0", seed=0, layers=args.layers)
        c5 = config5_prefix(args, model, args.batch)
        print(json.dumps(dict(metric=METRIC, n_gpus=1, dtype=DTYPE, data=DATA, higher_is_better=True,
                              config={"workload": c5["workload"]}, **c5)), flush=True)
        return 0
    headroom = args.warmup + 1 + GRAPH_WARMUP + args.steps + args.kernel_steps + 2
    d = Decoder(shape, args.batch, args.ctx_lo, args.ctx_hi, args.pool_blocks, headroom, layers=args.layers,
                kv_layout=args.kv_layout, fuse_mlp=args.fuse_mlp)
    if args.workload == "attention":
        c2 = config2_attention(args, d.pool, d.n_layers)
        print(json.dumps({"metric": "paged decode attention algorithmic HBM GB/s (config 2)", "value": c2["gbps"],
                          "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "dtype": DTYPE, "data": DATA,
                          "config": {"workload": c2["workload"]}, **c2}), flush=True)
        return 0
    out = headline(args, d)
    done("headline step")
    if args.workload == "all":
        configs = {}
        configs["config2_attention"] = config2_attention(args, d.pool, d.n_layers)
        done("config 2")
        configs["config5_prefix_batch"] = config5_prefix(args, d.model)
        done("config 5")
        del d
        torch.cuda.empty_cache()
        configs["config3_qwen2_0.5b"] = config3_qwen(args)
        done("config 3")
        configs["config1_linear"], configs["config4_linear_sweep"] = config14_linears(args)
        done("configs 1 and 4")
        out["configs"] = configs
        out["wall_s"] = round(time.perf_counter() - t_start, 1)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
