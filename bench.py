"""Throughput of the quantized Qwen2.5-1.5B decoder-layer hot path on one MI355X.

The default run measures the whole metric (decode tok/s and prefill tok/s, with their rooflines) and
prints ONE JSON line:
  value     28-layer Qwen2.5-1.5B-shaped batched decode, 64 sequences, each with a 4096-position KV
            history (K/V N(0,1), INT4 quantize/dequantize per row) and one new random token per step,
            positions 4096..4127 (32 steps, then the cycle repeats); a step is one decode token for
            all 64 sequences through all 28 layers (embedding gather + 28 x [RMSNorm, QKV, RoPE + KV
            append, GQA attention, O, RMSNorm, gate/up + SiLU, down + residual, bf16 rounding]);
  prefill   28-layer prefill of 8 independent sequences x 2048 random tokens (causal, full KV cache);
  greedy    28-layer batch-1 greedy generation: a 512-token prompt prefilled, then 128 decode steps
            through the final RMSNorm, the tied bf16 lm_head and argmax, all on the device.
Weights are random-init N(0, 0.02), rounded to bf16 and quantized per row to INT4 on the device
(seeds 4, 3 and 2).  Each part carries its dominant kernel's roofline (HIP events on the stream the
kernel runs on) and the reference's CPU path timed on this machine's host cores on a bounded sample.

    python bench.py [--steps K] [--warmup W] [--workload all|decode64|decode1|prefill] [--mode fast|ordered]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s & prefill tok/s (Qwen2.5-1.5B shapes, 1 GPU), % of roofline"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
LAYERS = 28
KV_ROW_BYTES = 1024  # 256 fp32 per token per layer, for K and again for V


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--workload", default="all", choices=["all", "decode64", "decode1", "prefill"])
    ap.add_argument("--mode", default="fast", choices=["fast", "ordered"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of each CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


# ---------------------------------------------------------------------------------------------
# CPU baseline: the reference decode host library compiled from the reference sources
# (oracle/_ref, built by oracle/Makefile), or the oracle restatement when it is absent.
# ---------------------------------------------------------------------------------------------
def cpu_baseline_decode(past: int, budget_s: float) -> dict:
    from work_llm_accelerator_amd.abi import SIGNATURES
    from work_llm_accelerator_amd.layout import HIDDEN, KV_WIDTH, LAYOUT
    from work_llm_accelerator_amd.quant import layer_views

    ref = ROOT / "oracle" / "_ref" / "libqwen_decode_ref.so"
    port = ROOT / "oracle" / "build" / "libqwen_oracle.so"
    if ref.exists():
        lib, name, kind = ctypes.CDLL(str(ref)), "qwen_decode_layer_smoke_forward", "reference"
    else:
        if not port.exists():
            os.system(f"make -s -C {ROOT / 'oracle'} oracle >/dev/null 2>&1")
        lib, name, kind = ctypes.CDLL(str(port)), "oracle_decode_layer_smoke_forward", "port"
    fn = getattr(lib, name)
    fn.argtypes = SIGNATURES["qwen_decode_layer_smoke_forward"]
    fn.restype = ctypes.c_int
    rng = np.random.default_rng(0)
    w = rng.integers(0, 256, LAYOUT.total_parameter_bytes, dtype=np.uint8)
    s = np.full((LAYOUT.total_parameter_bytes + 3) // 4, 0.01, np.float32)
    v = layer_views(w, s)
    v["input_layernorm"][:] = 1.0
    v["post_attention_layernorm"][:] = 1.0
    args = [v[k] for k in ("input_layernorm", "post_attention_layernorm", "q_w", "k_w", "v_w", "o_w", "gate_w",
                           "up_w", "down_w", "q_bias", "k_bias", "v_bias", "q_s", "k_s", "v_s", "o_s", "gate_s",
                           "up_s", "down_s")]
    x = rng.standard_normal(HIDDEN, dtype=np.float32)
    kc = rng.standard_normal((past + 1) * KV_WIDTH, dtype=np.float32)
    vc = rng.standard_normal((past + 1) * KV_WIDTH, dtype=np.float32)
    out = np.zeros(HIDDEN, np.float32)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        st = fn(x, past, *args, kc, vc, out)
        times.append(time.perf_counter() - t0)
        if st != 0:
            raise RuntimeError(f"CPU baseline returned {st}")
    t_layer = float(np.median(times))
    return {"value": 1.0 / (LAYERS * t_layer), "unit": "tok/s", "cores": 1, "kind": kind, "per_sequence": True,
            "sample": f"{len(times)} single-layer decode steps of one sequence at KV length {past + 1} through "
                      f"{'the reference decode .so built from its sources' if kind == 'reference' else 'the oracle'}"
                      f" (median {t_layer * 1e3:.1f} ms/layer-token, 1 thread), extrapolated x{LAYERS} layers. "
                      f"The reference decodes one sequence at a time, so this per-sequence rate is also its "
                      f"throughput on a batch; CPU: {cpu_model()}, {os.cpu_count()} visible cores"}


def cpu_baseline_prefill(seq: int, budget_s: float) -> dict:
    """The reference prefill arithmetic on one host core: the oracle's restatement (the reference
    prefill library needs Catapult's ac_channel.h and cannot be built here), one layer of `seq`
    tokens per call, extrapolated x28 layers."""
    from work_llm_accelerator_amd.layout import HIDDEN, KV_WIDTH, LAYOUT

    port = ROOT / "oracle" / "build" / "libqwen_oracle.so"
    if not port.exists():
        os.system(f"make -s -C {ROOT / 'oracle'} oracle >/dev/null 2>&1")
    lib = ctypes.CDLL(str(port))
    f32 = np.ctypeslib.ndpointer(dtype=np.float32, ndim=1, flags="C_CONTIGUOUS")
    u8 = np.ctypeslib.ndpointer(dtype=np.uint8, ndim=1, flags="C_CONTIGUOUS")
    fn = lib.oracle_prefill_layer_uncapped
    fn.argtypes = [f32, ctypes.c_int, u8, f32, f32, f32, f32]
    fn.restype = ctypes.c_int
    rng = np.random.default_rng(0)
    w = rng.integers(0, 256, LAYOUT.total_parameter_bytes, dtype=np.uint8)
    sc = np.full((LAYOUT.total_parameter_bytes + 3) // 4, 0.01, np.float32)
    x = rng.standard_normal(seq * HIDDEN, dtype=np.float32)
    kc = np.zeros(seq * KV_WIDTH, np.float32)
    vc = np.zeros(seq * KV_WIDTH, np.float32)
    out = np.zeros(seq * HIDDEN, np.float32)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        if fn(x, seq, w, sc, kc, vc, out) != 0:
            raise RuntimeError("CPU prefill baseline failed")
        times.append(time.perf_counter() - t0)
    t_call = float(np.median(times))
    return {"value": seq / (LAYERS * t_call), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} single-layer prefills of {seq} tokens (the reference's per-call cap) through "
                      f"the oracle restatement of the reference prefill arithmetic (median {t_call:.2f} s per call, "
                      f"1 thread), extrapolated x{LAYERS} layers; at 2048 tokens the causal attention adds about "
                      f"10% per token that this sample does not include; CPU: {cpu_model()}, "
                      f"{os.cpu_count()} visible cores"}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------------------------
TRAFFIC_PROFILE = ROOT / "profiles" / "attn_decode_b64_kv4096_hbm_traffic.json"
GREEDY_TRAFFIC = ROOT / "profiles" / "greedy_b1_prompt512_hbm_traffic.json"
PREFILL_TRAFFIC = ROOT / "profiles" / "prefill_8x2048_hbm_traffic.json"


def measured_traffic(batch: int, history: int):
    """HBM bytes per launch of the decode attention kernel at 64 sequences x KV 4096, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes (each scaled by the same counter's reading
    for a 1 GiB copy); None for other shapes or when the summary is absent."""
    if (batch, history) != (64, 4096) or not TRAFFIC_PROFILE.exists():
        return None
    return json.loads(TRAFFIC_PROFILE.read_text())["traffic_bytes_per_launch"]


def profiled_traffic(profile: Path, step: str):
    """HBM bytes per launch of one step of a workload, from its committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (copy-calibrated like measured_traffic); None when the summary is absent."""
    if not profile.exists():
        return None
    return json.loads(profile.read_text())["kernels"][step]["traffic_bytes_per_launch"]


def copy_bandwidth(torch, nbytes: int = 1 << 30, reps: int = 5) -> dict:
    """Device-to-device copy of `nbytes` (torch's copy kernel): the measured stream bandwidth of this
    GPU, and the kernel of known size whose HBM counters (FETCH_SIZE, WRITE_SIZE) scale the traffic."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    torch.cuda.empty_cache()
    return {"GBs": 2 * nbytes / (ms * 1e-3) / 1e9, "bytes_read": nbytes, "bytes_written": nbytes, "avg_us": ms * 1e3}


def bench_decode(args, torch, batch: int, history: int, seed: int) -> dict:
    from work_llm_accelerator_amd.model import (KERNEL_ATTN_DECODE, KERNEL_GEMM_DOWN, KERNEL_GEMM_GATE_UP,
                                                MODE_FAST, MODE_ORDERED, DeviceModel, KvCache, fill_kv_synthetic)

    mode = MODE_FAST if args.mode == "fast" else MODE_ORDERED
    cycle = 32
    positions = history + cycle
    model = DeviceModel(LAYERS, synthetic_seed=seed)
    cache = KvCache.allocate(LAYERS, batch, positions)
    fill_kv_synthetic(cache, seed + 1000)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    nsteps = args.warmup + args.steps
    ids = torch.randint(0, 151936, (nsteps, batch), dtype=torch.int32, device="cuda", generator=gen)
    pos = [torch.full((batch,), history + (i % cycle), dtype=torch.int32, device="cuda") for i in range(cycle)]
    hidden = torch.empty(batch, 1536, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        model.embed(ids[i], hidden, order=False)
        model.decode(mode, hidden, pos[i % cycle], positions, cache, order=False)

    for i in range(args.warmup):
        step(i)
    model.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(model.stream)
    for i in range(args.warmup, nsteps):
        step(i)
    e1.record(model.stream)
    model.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1)
    ms_step = ev_ms / args.steps
    last_pos = history + ((nsteps - 1) % cycle)
    keys = last_pos + 1
    res = {"value": batch * args.steps / (ev_ms / 1e3), "ms_per_step": ms_step, "wall_s": wall}
    # algorithmic bytes of one step (all layers): INT4 weights + fp32 norms/biases/scales, KV read
    # (keys rows of K and V) + the appended row, activations in/out.
    param_bytes = 23_508_992
    kv_read = batch * keys * 2 * KV_ROW_BYTES
    step_bytes = LAYERS * (param_bytes + kv_read + batch * 2 * KV_ROW_BYTES + batch * 2 * 1536 * 4)
    res["step_roofline"] = {"bound": "hbm", "algorithmic_bytes": step_bytes,
                            "achieved_GBs": step_bytes / (ms_step * 1e-3) / 1e9,
                            "frac": step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS}
    if mode == MODE_FAST:
        # dominant kernel: decode attention over the KV cache (96% of the step's bytes at 64 x 4096),
        # including its fused split merge and O-projection input quantization
        attn_ms = model.time_kernel(KERNEL_ATTN_DECODE, 0, 20)
        attn_bytes = kv_read + batch * 1536 * 4
        res["roofline"] = {"bound": "hbm", "kernel": "attn_decode_kernel", "achieved":
                           attn_bytes / (attn_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": attn_bytes / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                           "traffic": measured_traffic(batch, history),
                           "avg_launch_us": attn_ms * 1e3, "algorithmic_bytes_per_launch": attn_bytes}
        gu_ms = model.time_kernel(KERNEL_GEMM_GATE_UP, 0, 20)
        dn_ms = model.time_kernel(KERNEL_GEMM_DOWN, 0, 20)
        gu_bytes = 2 * 8960 * 1536 // 2 + 2 * 8960 * 4 + batch * 1536 * 2 + batch * 8960 * 4
        dn_bytes = 1536 * 8960 // 2 + 1536 * 4 + batch * 8960 * 2 + 2 * batch * 1536 * 4
        res["kernels"] = {
            "gemm_gate_up": {"avg_us": gu_ms * 1e3, "GBs": gu_bytes / (gu_ms * 1e-3) / 1e9},
            "gemm_down": {"avg_us": dn_ms * 1e3, "GBs": dn_bytes / (dn_ms * 1e-3) / 1e9},
        }
    model.close()
    del cache
    torch.cuda.empty_cache()
    return res


def bench_greedy(args, torch, prompt: int, seed: int) -> dict:
    """Batch-1 greedy generation: a `prompt`-token prompt of uniform random ids is prefilled, its last
    position's greedy token starts the loop, then each timed step is embedding -> 28 layers -> final
    RMSNorm -> tied bf16 lm_head -> argmax -> the next step's token, all on the device."""
    from work_llm_accelerator_amd.model import MODE_FAST, MODE_ORDERED, DeviceModel, KvCache

    mode = MODE_FAST if args.mode == "fast" else MODE_ORDERED
    nsteps = args.warmup + args.steps
    positions = prompt + nsteps
    model = DeviceModel(LAYERS, synthetic_seed=seed)
    vocab = model.vocab
    cache = KvCache.allocate(LAYERS, 1, positions)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    prompt_ids = torch.randint(0, vocab, (prompt,), dtype=torch.int32, device="cuda", generator=gen)
    hp = torch.empty(1, prompt, 1536, dtype=torch.float32, device="cuda")
    ids = torch.empty(1, dtype=torch.int32, device="cuda")
    hidden = torch.empty(1, 1536, dtype=torch.float32, device="cuda")
    pos = [torch.full((1,), prompt + i, dtype=torch.int32, device="cuda") for i in range(nsteps)]
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(model.stream)
    model.embed(prompt_ids, hp, order=False)
    model.prefill(mode, hp, cache, order=False)
    model.greedy(hp[0, prompt - 1:], ids, order=False)
    e1.record(model.stream)
    model.synchronize()
    prefill_ms = e0.elapsed_time(e1)

    def step(i):
        model.embed(ids, hidden, order=False)
        model.decode(mode, hidden, pos[i], positions, cache, order=False)
        model.greedy(hidden, ids, order=False)

    for i in range(args.warmup):
        step(i)
    model.synchronize()
    t0 = time.perf_counter()
    e0.record(model.stream)
    for i in range(args.warmup, nsteps):
        step(i)
    e1.record(model.stream)
    model.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    keys = prompt + nsteps  # KV rows read by the last step
    table_bytes = vocab * 1536 * 2
    res = {"value": 1.0 / (ms_step * 1e-3), "ms_per_step": ms_step, "wall_s": wall,
           "prefill": {"prompt_tokens": prompt, "ms": prefill_ms, "tok_s": prompt / (prefill_ms * 1e-3)}}
    step_bytes = LAYERS * (23_508_992 + keys * 2 * KV_ROW_BYTES + 2 * KV_ROW_BYTES + 2 * 1536 * 4) + table_bytes
    res["step_roofline"] = {"bound": "hbm", "algorithmic_bytes": step_bytes, "note": "includes the bf16 lm_head",
                            "achieved_GBs": step_bytes / (ms_step * 1e-3) / 1e9,
                            "frac": step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS}
    # dominant kernel: the lm_head streaming the bf16 table (its norm and argmax kernels included)
    reps = 20
    e0.record(model.stream)
    for _ in range(reps):
        model.greedy(hidden, ids, order=False)
    e1.record(model.stream)
    model.synchronize()
    head_ms = e0.elapsed_time(e1) / reps
    head_bytes = table_bytes + 1536 * 4 + 1536 * 2
    res["roofline"] = {"bound": "hbm", "kernel": "lm_head_row_kernel (with head_norm_kernel and argmax_finalize_kernel)",
                       "achieved": head_bytes / (head_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": head_bytes / (head_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                       "traffic": profiled_traffic(GREEDY_TRAFFIC, "lm_head (bf16 table)"),
                       "avg_launch_us": head_ms * 1e3, "algorithmic_bytes_per_launch": head_bytes}
    model.close()
    del cache
    torch.cuda.empty_cache()
    return res


def bench_prefill(args, torch, batch: int, seq: int, seed: int) -> dict:
    from work_llm_accelerator_amd.model import (KERNEL_ATTN_PREFILL, KERNEL_GEMM_GATE_UP, MODE_FAST, MODE_ORDERED,
                                                DeviceModel, KvCache)

    mode = MODE_FAST if args.mode == "fast" else MODE_ORDERED
    model = DeviceModel(LAYERS, synthetic_seed=seed)
    cache = KvCache.allocate(LAYERS, batch, seq)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    ids = torch.randint(0, 151936, (batch * seq,), dtype=torch.int32, device="cuda", generator=gen)
    hidden = torch.empty(batch, seq, 1536, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def step():
        model.embed(ids, hidden, order=False)
        model.prefill(mode, hidden, cache, order=False)

    for _ in range(args.warmup):
        step()
    model.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(model.stream)
    for _ in range(args.steps):
        step()
    e1.record(model.stream)
    model.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    tokens = batch * seq
    macs = LAYERS * (46_792_704 * tokens + batch * 12 * 128 * seq * (seq + 1))  # projections + QK^T, PV (causal)
    res = {"value": tokens / (ms * 1e-3), "ms_per_step": ms,
           "step_roofline": {"bound": "mfma", "algorithmic_TOPs": 2 * macs / 1e12,
                             "achieved_TOPs": 2 * macs / (ms * 1e-3) / 1e12,
                             "frac_int8": 2 * macs / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS}}
    if mode == MODE_FAST:
        gu_ms = model.time_kernel(KERNEL_GEMM_GATE_UP, 0, 5)
        at_ms = model.time_kernel(KERNEL_ATTN_PREFILL, 0, 5)
        gu_ops = 2 * 2 * 8960 * 1536 * tokens
        res["roofline"] = {"bound": "mfma", "kernel": "gemm_i8_pipe_kernel (gate/up + SiLU·up)",
                           "achieved": gu_ops / (gu_ms * 1e-3) / 1e12, "peak": INT8_PEAK_TOPS,
                           "unit": "TOP/s (int8 dense)", "frac": gu_ops / (gu_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                           "traffic": profiled_traffic(PREFILL_TRAFFIC, "gate/up + SiLU·up"),
                           "avg_launch_us": gu_ms * 1e3,
                           "issued_frac": 2 * gu_ops / (gu_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                           "note": "algorithmic ops; the two-limb code issues 2 int8 MFMA products per weight x "
                                   "activation product (issued_frac); MFMA busy cycles from counters in "
                                   "profiles/prefill_8x2048_mfma_utilisation.md"}
        res["kernels"] = {"attn_prefill": {"avg_us": at_ms * 1e3}}
    model.close()
    return res


def decode64_config():
    return {"workload": "28-layer Qwen2.5-1.5B-shaped batched decode: 64 sequences x KV history 4096 (positions "
                        "4096..4127), 1 new random token per sequence per step, seed 4",
            "layers": LAYERS, "batch": 64, "kv_length": "4097..4128"}


def prefill_config():
    return {"workload": "28-layer Qwen2.5-1.5B-shaped prefill: 8 sequences x 2048 random tokens, causal, full KV "
                        "cache written, seed 3", "layers": LAYERS, "batch": 8, "seq_len": 2048}


def greedy_config(args, steps):
    return {"workload": "28-layer Qwen2.5-1.5B-shaped greedy generation, batch 1: a 512-token prompt of uniform "
                        f"random ids prefilled, then {steps} greedy decode steps (embedding, 28 layers, final RMSNorm, "
                        "tied bf16 lm_head over 151936 tokens, argmax), seed 2", "layers": LAYERS, "batch": 1,
            "prompt": 512, "kv_length": f"{512 + args.warmup + 1}..{512 + args.warmup + steps}"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box of this run has one MI355X and the hot path needs no "
              f"collective (sequences shard data-parallel with no exchange); --gpus {args.gpus} is not run.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no GPU visible)", file=sys.stderr)
        sys.exit(1)
    dtype = "int4 weights x int8 two-limb MFMA, f32" if args.mode == "fast" else "f32"
    common = {"n_gpus": 1, "warmup": args.warmup, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
              "dtype": dtype, "data": "synthetic (random-init weights, random tokens, N(0,1) quantized KV)"}

    def part(r, config, steps):
        d = {"value": r["value"], "unit": "tok/s", "steps": steps, "ms_per_step": r["ms_per_step"],
             "config": {**config, "mode": args.mode}}
        for k in ("roofline", "step_roofline", "kernels", "prefill"):
            if k in r:
                d[k] = r[k]
        return d

    greedy_steps = 128
    if args.workload in ("all", "decode64"):
        r = bench_decode(args, torch, 64, 4096, 4)
        line = {"metric": METRIC, **part(r, decode64_config(), args.steps), **common}
        if args.workload == "all":
            pr = bench_prefill(argparse.Namespace(**{**vars(args), "steps": max(3, min(args.steps, 8)),
                                                     "warmup": min(args.warmup, 2)}), torch, 8, 2048, 3)
            line["prefill"] = part(pr, prefill_config(), max(3, min(args.steps, 8)))
            gr = bench_greedy(argparse.Namespace(**{**vars(args), "steps": greedy_steps}), torch, 512, 2)
            line["greedy"] = part(gr, greedy_config(args, greedy_steps), greedy_steps)
    elif args.workload == "decode1":
        r = bench_greedy(args, torch, 512, 2)
        line = {"metric": METRIC, **part(r, greedy_config(args, args.steps), args.steps), **common}
    else:
        r = bench_prefill(args, torch, 8, 2048, 3)
        line = {"metric": METRIC, **part(r, prefill_config(), args.steps), **common}
    line["copy_bandwidth"] = copy_bandwidth(torch)
    if not args.no_cpu:
        if args.workload in ("all", "decode64"):
            line["cpu_baseline"] = cpu_baseline_decode(4096, args.cpu_seconds)
        if args.workload == "all":
            line["prefill"]["cpu_baseline"] = cpu_baseline_prefill(128, args.cpu_seconds / 2)
            line["greedy"]["cpu_baseline"] = cpu_baseline_decode(576, args.cpu_seconds / 2)
            line["greedy"]["cpu_baseline"]["sample"] += " (the lm_head is not included)"
        elif args.workload == "decode1":
            line["cpu_baseline"] = cpu_baseline_decode(576, args.cpu_seconds)
        else:
            line["cpu_baseline"] = cpu_baseline_prefill(128, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
