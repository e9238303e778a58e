"""Benchmark of the KDA mixer hot path on one MI355X.

Headline workload (the value of the JSON line): chunk-64 KDA prefill over a
packed ragged batch -- 8 sequences with lengths uniform in [256, 4096]
(seeded), 16 heads x 128, bf16 q/k/v/o, fp32 log-decay g in [-5, 0], fp32
beta = sigmoid(N(0,1)), fp32 state, zero initial state.  One step = one
``sophia_kda_chunk_fwd`` call (intra-chunk + scan kernels) over the
whole batch with inputs resident in HBM and the host copy of the offsets
passed (FlashKDA's cu_seqlens_cpu), timed as eager calls and as HIP-graph
replays of 10 calls; the faster is the figure (the eager events also hold
the GPU's wait for the host to issue each call).

Also reported: the batch-256 decode step (fp32 state N(0, 0.02), one bf16
token per sequence) in microseconds and HBM GB/s (launched eagerly and as
HIP-graph replays of 10 steps; the faster is the headline figure), the ShortConv prefill over
the same packed batch (timed the same two ways), and the CPU baseline (the C restatement of the
reference's per-token recurrence, timed on this host's cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

HEADS, DIM, CHUNK = 16, 128, 64
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# Algorithmic traffic of the prefill core per token: q, k, v, o bf16 + g fp32
# + beta fp32 over 16 heads.
PREFILL_BYTES_PER_TOKEN = HEADS * (4 * DIM * 2 + DIM * 4 + 4)          # 24,640
# Causal chunk-form flops per token at C = 64: H * (5 C d + 6 d^2).
PREFILL_FLOPS_PER_TOKEN = HEADS * (5 * CHUNK * DIM + 6 * DIM * DIM)   # 2,228,224
METRIC = "KDA prefill tokens/s + % MFMA peak; decode-step µs and HBM GB/s at B=256"
# HBM bytes per launch come from the rocprofv3 counter summary committed under
# profiles/ (FETCH_SIZE and WRITE_SIZE in separate passes, calibrated on a plain
# 1 GiB device copy); the summary carries them in a fenced ```json block with
# the kernel build they were measured on.  Missing figures are reported as null.
TRAFFIC_PROFILE = os.path.join(HERE, "profiles", "hbm_traffic_counters.md")


def measured_traffic() -> dict:
    """{"bytes": {workload: bytes per call}, "source": ...} parsed from the
    counter summary, or empty figures when it is absent."""
    try:
        text = open(TRAFFIC_PROFILE).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        data = json.loads(block)
        return {"bytes": data.get("traffic_bytes_per_call", {}),
                "source": f"profiles/hbm_traffic_counters.md ({data.get('measured', 'undated')})"}
    except (OSError, IndexError, ValueError):
        return {"bytes": {}, "source": None}


def prefill_lengths(seed: int = 0, n: int = 8, lo: int = 256, hi: int = 4096) -> list[int]:
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=n)]


def make_prefill_inputs(torch, dev, lengths, seed=1):
    gen = torch.Generator().manual_seed(seed)
    total = int(sum(lengths))
    shape = (total, HEADS, DIM)
    q = torch.nn.functional.normalize(torch.randn(shape, generator=gen), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn(shape, generator=gen), dim=-1).to(torch.bfloat16)
    v = torch.randn(shape, generator=gen).to(torch.bfloat16)
    g = torch.rand(shape, generator=gen) * -5.0
    beta = torch.sigmoid(torch.randn((total, HEADS), generator=gen))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    inputs = {name: t.to(dev) for name, t in dict(q=q, k=k, v=v, g=g, beta=beta, cu=cu).items()}
    inputs["cu_cpu"] = cu  # the host copy of the offsets (FlashKDA's cu_seqlens_cpu)
    return inputs


def graph_ms_per_call(torch, dev, fn, replays: int, stream, per_graph: int = 10) -> float:
    """Average duration (ms) of one call of `fn` when `per_graph` calls are
    captured in a HIP graph (after a warm-up on the capture stream) and the
    graph is replayed: the events then bracket the kernels alone."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    with torch.cuda.graph(graph, stream=side):
        for _ in range(per_graph):
            fn()
    _, per = time_events(torch, graph.replay, replays, 2, stream)
    del graph
    return float(np.mean(per)) / per_graph


def time_events(torch, fn, steps: int, warmup: int, stream) -> tuple[float, list[float]]:
    """Average per-call duration (ms) from HIP events recorded on `stream`
    around each call, plus the wall time of the whole timed region."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return wall, per


def cpu_baseline(inputs, lengths, budget_s: float = 10.0):
    """The oracle's C restatement of the reference's per-token recurrence
    (oracle/kda_ref.c, fp32, OpenMP over sequence x head) on this host's
    cores, over the same packed batch, repeated until about `budget_s`
    seconds of CPU work have been timed."""
    from oracle import c_oracle
    cores = len(os.sched_getaffinity(0))
    q = inputs["q"].float().cpu().numpy()
    k = inputs["k"].float().cpu().numpy()
    v = inputs["v"].float().cpu().numpy()
    g = inputs["g"].cpu().numpy()
    beta = inputs["beta"].cpu().numpy()
    cu = inputs["cu"].cpu().numpy()
    reps, elapsed = 0, 0.0
    while elapsed < budget_s:
        t0 = time.perf_counter()
        c_oracle.kda_varlen(q, k, v, g, beta, cu, use_gate=False, use_beta_sigmoid=False,
                            nthreads=cores)
        elapsed += time.perf_counter() - t0
        reps += 1
    tokens = int(cu[-1])
    return {"value": round(tokens * reps / elapsed, 1), "unit": "tokens/s", "cores": cores,
            "kind": "port",
            "sample": f"whole workload ({tokens} tokens x 16 heads) run {reps} times in "
                      f"{elapsed:.1f} s by the C per-token fp32 recurrence of the reference's "
                      f"CPU path (OpenMP over sequence x head, {cores} threads); "
                      f"os.cpu_count()={os.cpu_count()}"}


def _threads(torch) -> dict:
    return {"os_cpu_count": os.cpu_count(), "affinity_cores": len(os.sched_getaffinity(0)),
            "torch_threads": torch.get_num_threads()}


def _timed(fn, budget_s: float, min_reps: int = 1) -> tuple[int, float]:
    reps, elapsed = 0, 0.0
    while elapsed < budget_s or reps < min_reps:
        t0 = time.perf_counter()
        fn()
        elapsed += time.perf_counter() - t0
        reps += 1
    return reps, elapsed


def cpu_baselines(torch, budget_s: float = 4.0) -> dict:
    """The reference's CPU path for the other configurations, restated by the
    oracle and timed on this host (fp32 throughout):
      config 1: the whole mixer layer (numpy restatement of SophiaKDA.forward,
                B = 1, T = 512, dim 1536, seed-42 init draws), ms per forward;
      config 3: one decode step of 256 sequences (C per-token recurrence,
                OpenMP over sequence x head, plus the conv step), us per step;
      config 4: the first 8,192 tokens of the 65,536-token sequence (C
                recurrence, 16 (sequence, head) pairs in parallel), tokens/s."""
    from oracle import c_oracle
    from oracle import kda_oracle as ko
    cores = len(os.sched_getaffinity(0))
    out = {}
    # config 1
    from sophia_amd.config import ModelArgs
    from sophia_amd.kda import SophiaKDA
    torch.manual_seed(42)
    params = {k: v.detach().numpy() for k, v in SophiaKDA(ModelArgs(max_batch_size=1)).state_dict().items()}
    x = np.random.default_rng(0).standard_normal((1, 512, 1536)).astype(np.float32)
    reps, el = _timed(lambda: ko.mixer_forward(params, x, num_heads=16), budget_s)
    out["config1_mixer_layer"] = {
        "value": round(el / reps * 1e3, 1), "unit": "ms/forward", "cores": cores, "kind": "port",
        "sample": f"B=1, T=512, dim 1536 forward run {reps} times: numpy restatement of "
                  f"SophiaKDA.forward in fp32 (BLAS GEMMs on the host's threads, the per-token "
                  f"recurrence serial)", **_threads(torch)}
    # config 3
    rng = np.random.default_rng(3)
    b, h = 256, 16
    q = rng.standard_normal((b, h, 128)).astype(np.float32)
    k = rng.standard_normal((b, h, 128)).astype(np.float32)
    v = rng.standard_normal((b, h, 128)).astype(np.float32)
    g = rng.uniform(-5.0, 0.0, (b, h, 128)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((b, h))))).astype(np.float32)
    s0 = (rng.standard_normal((b, h, 128, 128)) * 0.02).astype(np.float32)
    cu = np.arange(b + 1, dtype=np.int32)
    xc = rng.standard_normal((b, 1, 3 * h * 128)).astype(np.float32)
    wc = (rng.standard_normal((3 * h * 128, 4)) * 0.02).astype(np.float32)
    hist = rng.standard_normal((b, 3 * h * 128, 3)).astype(np.float32)

    def decode():
        ko.short_conv(xc, wc, hist)
        c_oracle.kda_varlen(q, k, v, g, beta, cu, initial_states=s0, use_gate=False,
                            use_beta_sigmoid=False, nthreads=cores)

    reps, el = _timed(decode, budget_s)
    out["config3_decode_step"] = {
        "value": round(el / reps * 1e6, 1), "unit": "us/step", "cores": cores, "kind": "port",
        "sample": f"B=256 one-token step run {reps} times: C per-token recurrence (OpenMP over 4,096 "
                  f"sequence x head pairs, {cores} threads) plus the numpy conv step", **_threads(torch)}
    # config 4
    t4 = 8192
    gen = torch.Generator().manual_seed(10)
    q4 = torch.nn.functional.normalize(torch.randn(t4, h, 128, generator=gen), dim=-1).numpy()
    k4 = torch.nn.functional.normalize(torch.randn(t4, h, 128, generator=gen), dim=-1).numpy()
    v4 = torch.randn(t4, h, 128, generator=gen).numpy()
    g4 = (torch.rand(t4, h, 128, generator=gen) * -4.5 - 0.5).numpy()
    b4 = torch.sigmoid(torch.randn(t4, h, generator=gen)).numpy()
    cu4 = np.array([0, t4], dtype=np.int32)
    reps, el = _timed(lambda: c_oracle.kda_varlen(q4, k4, v4, g4, b4, cu4, use_gate=False,
                                                  use_beta_sigmoid=False, nthreads=cores), budget_s)
    out["config4_long_prefill"] = {
        "value": round(t4 * reps / el, 1), "unit": "tokens/s", "cores": min(cores, h), "kind": "port",
        "sample": f"first 8,192 tokens of the 65,536-token sequence x 16 heads run {reps} times: C "
                  f"per-token recurrence, one thread per head (16 pairs)", **_threads(torch)}
    return out


def long_prefill_bench(torch, dev, stream, steps: int, warmup: int, traffic: dict) -> dict:
    """Config 4: one sequence of 65,536 tokens (1,024 chunks), 16 heads, bf16
    q/k/v/o, fp32 g ~ U[-5, -0.5] and beta, zero initial state, final state
    written; timed like the headline prefill."""
    from sophia_amd import ops
    total = 65536
    gen = torch.Generator().manual_seed(10)
    shape = (total, HEADS, DIM)
    q = torch.nn.functional.normalize(torch.randn(shape, generator=gen), dim=-1).to(torch.bfloat16).to(dev)
    k = torch.nn.functional.normalize(torch.randn(shape, generator=gen), dim=-1).to(torch.bfloat16).to(dev)
    v = torch.randn(shape, generator=gen).to(torch.bfloat16).to(dev)
    g = (torch.rand(shape, generator=gen) * -4.5 - 0.5).to(dev)
    beta = torch.sigmoid(torch.randn((total, HEADS), generator=gen)).to(dev)
    cu_cpu = torch.tensor([0, total], dtype=torch.int32)
    cu = cu_cpu.to(dev)
    final = torch.zeros((1, HEADS, DIM, DIM), device=dev)
    out = torch.empty(shape, dtype=torch.bfloat16, device=dev)

    def call():
        ops.kda_chunk_fwd(q, k, v, g, beta, cu, use_qk_l2norm=True, use_gate=False,
                          use_beta_sigmoid=False, final_state=final, out=out, cu_seqlens_cpu=cu_cpu)

    _, per = time_events(torch, call, steps, warmup, stream)
    eager = float(np.mean(per))
    graph = graph_ms_per_call(torch, dev, call, max(steps // 2, 3), stream, per_graph=4)
    ms = min(eager, graph)
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("non-finite long-prefill output")
    gbs = total * PREFILL_BYTES_PER_TOKEN / (ms / 1e3) / 1e9
    tflops = total * PREFILL_FLOPS_PER_TOKEN / (ms / 1e3) / 1e12
    return {"workload": "KDA chunk prefill, one sequence of 65,536 tokens (1,024 chunks), 16 heads x 128, "
                        "bf16 q/k/v/o, fp32 g ~ U[-5,-0.5] / beta / state",
            "tokens_per_s": round(total / (ms / 1e3), 1), "ms_per_call": round(ms, 4),
            "ms_eager": round(eager, 4), "ms_graph": round(graph, 4),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": traffic["bytes"].get("long_prefill"),
                         "traffic_source": traffic["source"],
                         "algorithmic_bytes_per_launch": total * PREFILL_BYTES_PER_TOKEN},
            "mfma": {"achieved_tflops": round(tflops, 2),
                     "frac_of_peak": round(tflops / BF16_PEAK_TFLOPS, 4)}}


# Backward bytes per (token, head): q, k, v, do in bf16 and g, beta in fp32 read;
# dq, dk, dv written in bf16 (the element type of q, k, v, as training takes
# them), dg and dbeta in fp32.
BWD_BYTES_PER_TOKEN = HEADS * (4 * DIM * 2 + DIM * 4 + 4 + 3 * DIM * 2 + DIM * 4 + 4)
# Backward flops per token of the chunk form (what the default backward runs),
# per chunk of C = 64 tokens and head, counting triangular products at half
# as the forward's 5 C^2 d + 6 C d^2 does:
#   records (the forward's intra phase): A_kk, A_qk, W = T (beta K e^G),
#     Ut = T (beta V): 4 C^2 d, and T = (I + A_kk)^-1: C^3 / 3;
#   forward states: U = Ut - W S0, S1 = D S0 + Kbar^T U: 4 C d^2;
#   reverse scan: dU = A_qk^T dO + Kbar dS1: C^2 d + 2 C d^2,
#     dS0 = D dS1 + Qg^T dO - W^T dU: 4 C d^2;
#   gradients: dA_qk = tril(dO U^T), Y = dU U^T (strictly lower),
#     dXu = T^T dU: 3 C^2 d; dA_kk = -T^T Y: C^3 / 3; dQg = dO S0^T,
#     dXw = -dXu S0^T, dKbar = U dS1^T: 6 C d^2; the products through A_qk
#     and P into dq^, dk^: 4 C^2 d.
# Total 12 C^2 d + 2 C^3 / 3 + 16 C d^2 per chunk and head (the split-bf16
# products of the gradient kernel issue three MFMAs per such product; only
# the useful flops are counted).
BWD_FLOPS_PER_TOKEN = HEADS * (12 * CHUNK * DIM + (2 * CHUNK * CHUNK) // 3 + 16 * DIM * DIM)


def backward_bench(torch, dev, stream, inp, steps: int, warmup: int, with_cpu: bool = False) -> dict:
    """The KDA backward (sophia_kda_chunk_bwd) over the headline prefill
    batch: gradients of q, k, v, g, beta and the initial states for a bf16
    output gradient, with the same flags as the timed prefill; dq, dk, dv in
    bf16 as the autograd function asks for them with bf16 q, k, v (the call
    with fp32 gradients is timed beside it)."""
    from sophia_amd import ops
    total = int(inp["q"].size(0))
    gen = torch.Generator().manual_seed(12)
    d_out = torch.randn((total, HEADS, DIM), generator=gen).to(torch.bfloat16).to(dev)

    def call(recurrent=False, grad_dtype=torch.bfloat16):
        ops.kda_chunk_bwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["cu"], d_out,
                          use_qk_l2norm=True, use_gate=False, use_beta_sigmoid=False,
                          cu_seqlens_cpu=inp["cu_cpu"], recurrent=recurrent, grad_dtype=grad_dtype)

    _, per = time_events(torch, call, steps, warmup, stream)
    ms_eager = float(np.mean(per))
    # As for the prefill: eager events also hold the gaps in which the GPU
    # waits for the host to issue each call's launches; graph replays bracket
    # the kernels alone.  The lower of the two is reported.
    ms_graph = graph_ms_per_call(torch, dev, call, max(steps // 2, 3), stream, per_graph=4)
    ms = min(ms_eager, ms_graph)
    ms_f32 = graph_ms_per_call(torch, dev, lambda: call(grad_dtype=torch.float32), max(steps // 2, 3), stream,
                               per_graph=4)
    _, per_rec = time_events(torch, lambda: call(True), max(steps // 2, 2), 1, stream)
    gbs = total * BWD_BYTES_PER_TOKEN / (ms / 1e3) / 1e9
    tflops = total * BWD_FLOPS_PER_TOKEN / (ms / 1e3) / 1e12
    out = {"workload": "KDA backward over the prefill batch (same lengths, flags and inputs), "
                       "bf16 d_out, bf16 dq / dk / dv, fp32 dg / dbeta / dh0",
           "form": "chunk (records, forward-state and reverse chunk scans on bf16 MFMA operands, "
                   "per-chunk gradients as split-bf16 MFMA products (hi*hi + hi*lo + lo*hi, fp32 "
                   "accumulation) with the norm, gate and sigmoid backward fused)",
           "tokens_per_s": round(total / (ms / 1e3), 1), "ms_per_call": round(ms, 3),
           "ms_eager": round(ms_eager, 3), "ms_graph": round(ms_graph, 3),
           "ms_graph_fp32_grads": round(ms_f32, 3),
           "recurrent_form_ms_per_call": round(float(np.mean(per_rec)), 3),
           "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                        "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                        "flops_per_token": BWD_FLOPS_PER_TOKEN,
                        "flops_convention": "the chunk form's useful flops, 12 C^2 d + 2 C^3 / 3 + 16 C d^2 "
                                            "per chunk and head (triangular products at half), against the "
                                            "bf16 dense MFMA peak its operands run at"},
           "algorithmic_bytes_per_call": total * BWD_BYTES_PER_TOKEN,
           "GBps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    if with_cpu:
        out["cpu_baseline"] = backward_cpu_baseline(torch, inp, d_out)
    return out


def backward_cpu_baseline(torch, inp, d_out, budget_s: float = 6.0) -> dict:
    """The oracle's C restatement of the backward (oracle/kda_ref.c: the
    chain rule through the reference's per-token recurrence, fp32, OpenMP
    over sequence x head) over the same batch on this host's cores."""
    from oracle import c_oracle
    cores = len(os.sched_getaffinity(0))
    args = [inp[n].float().cpu().numpy() for n in ("q", "k", "v", "g", "beta")]
    cu = inp["cu_cpu"].numpy()
    do = d_out.float().cpu().numpy()
    total = int(cu[-1])
    reps, el = _timed(lambda: c_oracle.kda_varlen_bwd(*args, cu, do, use_qk_l2norm=True, use_gate=False,
                                                      use_beta_sigmoid=False, nthreads=cores), budget_s)
    return {"value": round(total * reps / el, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"whole workload ({total} tokens x 16 heads) run {reps} times by the C backward "
                      f"of the per-token recurrence (OpenMP over sequence x head, {cores} threads)",
            **_threads(torch)}


def copy_bandwidth(torch, dev, stream, nbytes: int = 1 << 30) -> float:
    """Device-to-device copy rate (GB/s, read + write bytes) of a plain
    torch copy kernel on this GPU: the practical HBM ceiling beside the
    8 TB/s vendor figure."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    _, per = time_events(torch, lambda: dst.copy_(src), 10, 3, stream)
    return 2 * nbytes / (float(np.median(per)) / 1e3) / 1e9


def mixed_step_bench(torch, dev, stream, steps: int, warmup: int, seed: int = 4,
                     tune_gemms: str | None = None, gemms: str = "both") -> dict:
    """The whole hybrid decoder (28 layers [KDA, KDA, KDA, MLA] x 7, dim 1536,
    16 heads x 128, SiTU-GLU 3968, MLA ranks 384 / 128, vocab 65,536, tied;
    random init, bf16 GEMM weights, fp32 caches) in one continuous-batching
    step: 16 new sequences of 1,024 tokens prefilled together with one decode
    token for each of 240 running sequences (cached lengths U[1, 1023],
    seeded; random latent caches, zero recurrent state).  The step is
    captured in a HIP graph after two warm-up runs on a side stream and
    replayed; the eager step is timed beside it.  The library GEMMs run first
    with hipBLASLt's default per-shape heuristics, then with the per-shape
    selection of sophia_amd/gemm_tuning_gfx950.csv (torch TunableOp, no timing
    runs) when that file matches this software stack; the step figures are
    those of the faster of the two, and both are reported (``gemms``:
    "default" or "tuned" runs one of them only).  With ``tune_gemms``, the
    selection is timed here and written to that file."""
    from sophia_amd.config import ModelArgs
    from sophia_amd.decoder import MixedStepGraph, Transformer
    from sophia_amd.kda import RuntimeLinear

    P, T, D, L = 16, 1024, 240, 1024
    args = ModelArgs(max_batch_size=P + D, max_seq_len=2048)
    torch.manual_seed(seed)
    with torch.device(dev):
        model = Transformer(args)
    model.cast_weights_(torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(seed)
    for layer in model.layers:
        if layer.layer_type == "mla":
            layer.attn.latent_cache.normal_(generator=gen)
    cpu_gen = torch.Generator().manual_seed(seed)
    step = dict(
        prefill_ids=torch.randint(0, args.vocab_size, (P, T), generator=cpu_gen).to(dev),
        decode_ids=torch.randint(0, args.vocab_size, (D,), generator=cpu_gen).to(dev),
        prefill_slots=torch.arange(P, dtype=torch.int32).to(dev),
        decode_slots=torch.arange(P, P + D, dtype=torch.int32).to(dev),
        decode_pos=torch.randint(1, L, (D,), generator=cpu_gen).to(dev))

    def eager():
        with torch.no_grad():
            return model.forward_mixed(max_decode_len=L, **step)

    from sophia_amd import gemm_tuning

    def measure():
        _, eper = time_events(torch, eager, max(steps // 4, 3), 2, stream)
        graph = MixedStepGraph(model, P, T, D, L, warmup=2, example=step)
        _, gper = time_events(torch, graph.run, steps, warmup, stream)
        if not torch.isfinite(graph.logits.float()).all():
            raise RuntimeError("non-finite logits from the captured mixed step")
        del graph
        return float(np.mean(gper)), float(np.mean(eper))

    gemm_runs = {}
    if gemms in ("both", "default") and not tune_gemms:
        gemm_runs["default"] = measure()
    if tune_gemms:
        gemm_tuning.use_tuned_gemms(tune_gemms, tune=True)
        eager()  # times every GEMM shape of the step once
        gemm_runs["tuned"] = measure()
    elif gemms in ("both", "tuned") and gemm_tuning.use_tuned_gemms():
        gemm_runs["tuned"] = measure()
    gemm_tuning.use_default_gemms()
    if not gemm_runs:
        gemm_runs["default"] = measure()
    selection = min(gemm_runs, key=lambda k: gemm_runs[k][0])
    gms, ems = gemm_runs[selection]
    tokens = P * T + D

    # Work per step: every per-token GEMM (MLA k_up / v_up on prefill rows
    # only; decode rows attend in latent space), the last-token head, causal
    # MLA attention, the absorbed decode attention over L cached latents, and
    # the KDA chunk core on the prefill rows.  Decode recurrences (HBM-bound)
    # are not counted.
    h, d, r = args.num_heads, args.head_dim, args.mla_kv_rank
    flops = 0.0
    for layer in model.layers:
        for name, mod in layer.named_modules():
            if not isinstance(mod, RuntimeLinear) or name.endswith("query"):
                continue
            rows = P * T if name in ("attn.k_up", "attn.v_up") else tokens
            flops += 2.0 * rows * mod.weight.numel()
        if layer.layer_type == "mla":
            flops += 2.0 * P * h * T * T * d + D * h * 4.0 * (d * r + L * r)
        else:
            flops += P * T * PREFILL_FLOPS_PER_TOKEN
    flops += 2.0 * (P + D) * args.vocab_size * args.dim
    tflops = flops / (gms / 1e3) / 1e12
    out = {"workload": "hybrid decoder, 28 layers [KDA,KDA,KDA,MLA]x7, dim 1536, bf16, one "
                       "mixed step: 16x1024 prefill + 240x1 decode, HIP-graph replay",
           "tokens_per_step": tokens, "ms_per_step": round(gms, 3),
           "tokens_per_s": round(tokens / (gms / 1e3), 1),
           "eager_ms_per_step": round(ems, 3), "graph_speedup": round(ems / gms, 3),
           "approx_tflops": round(tflops, 1),
           "frac_of_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
           "flops_per_step": flops, "steps": steps,
           "gemm_selection": selection,
           "ms_per_step_by_gemm_selection": {k: round(v[0], 3) for k, v in gemm_runs.items()}}
    del model
    torch.cuda.empty_cache()
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--mixed-gemms", choices=["both", "default", "tuned"], default="both",
                    help="library GEMM selection(s) timed in the mixed step")
    ap.add_argument("--tune-gemms", metavar="CSV", default=None,
                    help="time the mixed step's library GEMM candidates and write the "
                         "per-shape selection to CSV (torch TunableOp)")
    ap.add_argument("--only", choices=["all", "kda", "prefill", "conv", "decode", "copy", "mixed", "long",
                                       "bwd"],
                    default="all",
                    help="run one workload only (for kernel profiling; 'kda' = prefill, ShortConv "
                         "and decode without the decoder step); the JSON line then carries that "
                         "workload's fields alone")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    from sophia_amd import ops, _native

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    _native.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)

    if args.only == "copy":
        # Calibration workload for the memory counters: a plain 1 GiB device copy.
        gbs = copy_bandwidth(torch, dev, stream)
        print(json.dumps({"metric": "device copy GB/s (read + write bytes)", "value": round(gbs, 1),
                          "unit": "GB/s", "bytes_read_per_copy": 1 << 30,
                          "bytes_written_per_copy": 1 << 30}), flush=True)
        return 0

    traffic = measured_traffic()
    lengths = prefill_lengths()
    total = int(sum(lengths))
    inp = make_prefill_inputs(torch, dev, lengths)
    final = torch.zeros((len(lengths), HEADS, DIM, DIM), dtype=torch.float32, device=dev)
    out = torch.empty((total, HEADS, DIM), dtype=torch.bfloat16, device=dev)

    def prefill():
        ops.kda_chunk_fwd(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["cu"],
                          use_qk_l2norm=True, use_gate=False, use_beta_sigmoid=False,
                          final_state=final, out=out, cu_seqlens_cpu=inp["cu_cpu"])

    result = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
              "data": "synthetic"}

    run_prefill = args.only in ("all", "kda", "prefill")
    wall, per = time_events(torch, prefill, args.steps if run_prefill else 1,
                            args.warmup if run_prefill else 0, stream)
    eager_ms = float(np.mean(per))
    graph_ms = eager_ms
    if run_prefill:
        # The same calls as replays of a HIP graph: the events then bracket the
        # kernels alone, without the host's time to issue each call (which the
        # eager events include when the GPU waits for it).
        graph_ms = graph_ms_per_call(torch, dev, prefill, max(args.steps // 2, 5), stream)
    avg_ms = min(eager_ms, graph_ms)
    tokens_per_s = total / (avg_ms / 1e3)
    achieved_gbs = total * PREFILL_BYTES_PER_TOKEN / (avg_ms / 1e3) / 1e9
    tflops = total * PREFILL_FLOPS_PER_TOKEN / (avg_ms / 1e3) / 1e12
    ai = PREFILL_FLOPS_PER_TOKEN / PREFILL_BYTES_PER_TOKEN
    attainable = min(BF16_PEAK_TFLOPS, HBM_PEAK_GBS * ai / 1e3)
    result.update({
        "value": round(tokens_per_s, 1), "unit": "tokens/s",
        "ms_per_step": round(wall / args.steps, 4),
        "config": {"workload": "KDA varlen chunk prefill (chunk 64): 8 sequences, lengths "
                               "U[256,4096] seed 0, 16 heads x 128, bf16 q/k/v/o, fp32 g in "
                               "[-5,0] / beta / state, zero initial state",
                   "lengths": lengths, "total_tokens": total, "heads": HEADS, "head_dim": DIM,
                   "kernel_ms": round(avg_ms, 4), "kernel_ms_eager": round(eager_ms, 4),
                   "kernel_ms_graph": round(graph_ms, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes"].get("prefill"), "traffic_source": traffic["source"],
                     "kernel": "kda_chunk_intra + kda_chunk_scan (one call)",
                     "algorithmic_bytes_per_launch": total * PREFILL_BYTES_PER_TOKEN},
        "mfma": {"achieved_tflops": round(tflops, 2), "peak_tflops": BF16_PEAK_TFLOPS,
                 "frac_of_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
                 "attainable_tflops": round(attainable, 1),
                 "frac_of_attainable": round(tflops / attainable, 4),
                 "flops_per_token": PREFILL_FLOPS_PER_TOKEN},
    })
    if not torch.isfinite(out.float()).all():
        print("non-finite prefill output", file=sys.stderr)
        return 1

    if not run_prefill:
        for key in ("value", "ms_per_step", "roofline", "mfma"):
            result.pop(key, None)

    # ShortConv over the same packed batch (3 x 2048 channels, bf16).
    gen = torch.Generator().manual_seed(2)
    xconv = torch.randn((total, 3 * HEADS * DIM), generator=gen).to(torch.bfloat16).to(dev)
    # taps rounded to the activation dtype once, as the decoder keeps them
    wconv = (torch.randn((3 * HEADS * DIM, 4), generator=gen) * 0.02).to(torch.bfloat16).float().to(dev)
    conv_state = torch.zeros((len(lengths), 3 * HEADS * DIM, 3), device=dev)
    yconv = torch.empty_like(xconv)

    def conv():
        ops.short_conv_fwd(xconv, wconv, inp["cu"], conv_state=conv_state, read_history=False,
                           write_history=True, out=yconv, weight_rounded=True)

    if args.only in ("all", "kda", "conv"):
        _, cper = time_events(torch, conv, args.steps, args.warmup, stream)
        ceager = float(np.mean(cper))
        cgraph = graph_ms_per_call(torch, dev, conv, max(args.steps // 2, 5), stream)
        cms = min(ceager, cgraph)
        cbytes = total * 3 * HEADS * DIM * 2 * 2
        result["short_conv"] = {"us": round(cms * 1e3, 2), "us_eager": round(ceager * 1e3, 2),
                                "us_graph": round(cgraph * 1e3, 2),
                                "GBps": round(cbytes / (cms / 1e3) / 1e9, 1),
                                "algorithmic_bytes": cbytes,
                                "traffic": traffic["bytes"].get("short_conv")}
    del xconv, yconv, conv_state

    # Decode step at B = 256.
    batch = 256
    gen = torch.Generator().manual_seed(3)
    shape = (batch, HEADS, DIM)
    dq = torch.nn.functional.normalize(torch.randn(shape, generator=gen), dim=-1).to(torch.bfloat16).to(dev)
    dk = torch.nn.functional.normalize(torch.randn(shape, generator=gen), dim=-1).to(torch.bfloat16).to(dev)
    dv = torch.randn(shape, generator=gen).to(torch.bfloat16).to(dev)
    dg = (torch.rand(shape, generator=gen) * -5.0).to(dev)
    db = torch.sigmoid(torch.randn((batch, HEADS), generator=gen)).to(dev)
    dstate = (torch.randn((batch, HEADS, DIM, DIM), generator=gen) * 0.02).to(dev)
    dout = torch.empty(shape, dtype=torch.bfloat16, device=dev)

    def decode():
        ops.kda_decode_step(dq, dk, dv, dg, db, dstate, use_gate=False, use_beta_sigmoid=False,
                            out=dout)

    if args.only in ("all", "kda", "decode"):
        dsteps = max(args.steps * 5, 50)
        _, dper = time_events(torch, decode, dsteps, args.warmup * 2, stream)
        eager_ms = float(np.mean(dper))
        # The same steps as a serving loop runs them: replays of a HIP graph of
        # 10 steps.
        graph_ms = graph_ms_per_call(torch, dev, decode, max(dsteps // 10, 5), stream)
        dms = min(eager_ms, graph_ms)
        dbytes = (2 * batch * HEADS * DIM * DIM * 4
                  + batch * HEADS * (3 * DIM * 2 + DIM * 4 + 4 + DIM * 2))
        dgbs = dbytes / (dms / 1e3) / 1e9
        result["decode"] = {"batch": batch, "us_per_step": round(dms * 1e3, 2),
                            "GBps": round(dgbs, 1),
                            "frac_of_hbm_peak": round(dgbs / HBM_PEAK_GBS, 4),
                            "us_per_step_eager": round(eager_ms * 1e3, 2),
                            "us_per_step_graph": round(graph_ms * 1e3, 2),
                            "algorithmic_bytes": dbytes, "steps": dsteps,
                            "traffic": traffic["bytes"].get("decode"),
                            "kernel": "kda_decode_kernel"}
    del dstate

    if args.only in ("all", "kda", "long"):
        result["long_prefill"] = long_prefill_bench(torch, dev, stream, max(args.steps // 2, 5),
                                                    max(args.warmup // 2, 2), traffic)
    if args.only in ("all", "bwd"):
        result["backward"] = backward_bench(torch, dev, stream, inp, max(args.steps // 4, 3),
                                            max(args.warmup // 2, 1), with_cpu=not args.no_cpu)
    if args.only in ("all", "mixed"):
        result["mixed_step"] = mixed_step_bench(torch, dev, stream, max(args.steps // 2, 5),
                                                max(args.warmup // 2, 2),
                                                tune_gemms=args.tune_gemms, gemms=args.mixed_gemms)
    if args.only == "all":
        result["hbm_copy_GBps"] = round(copy_bandwidth(torch, dev, stream), 1)
    if not args.no_cpu and args.only == "all":
        result["cpu_baseline"] = cpu_baseline(inp, lengths)
        result["cpu_baseline"].update(_threads(torch))
        result["cpu_baselines_other_configs"] = cpu_baselines(torch)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
