#!/usr/bin/env python3
"""Benchmark of the MI355X DiT hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--legs attention,sage] [--no-cpu]

Headline workload: BF16 DiT self-attention, S = 27x30x40 =
32400 tokens, B = 1, H = 40, D = 128, Q/K/V = 0.5 N(0,1) BF16 with the 3D RoPE
applied to Q and K. A "step" is one attention call over that input, resident in
HBM before the timed region. value = 4 S^2 H D / (time per call) in TFLOP/s.

Extra legs (own JSON objects on the same line): the Sage int8/fp8 attention on
config 3's inputs. The CPU baseline times the oracle's restatement of the
reference operator on a bounded sample (a slice of query rows, all keys and
heads) on the host cores and scales it to the same unit.
"""
import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np
from ctypes import c_float as C_float

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

SEQ, HEADS, DIM = 32400, 40, 128
ROPE_SHAPE = (27, 30, 40)
PEAK_BF16 = 2500.0      # MI355X dense BF16 MFMA, TFLOP/s
PEAK_FP8 = 5000.0       # MI355X dense FP8 / INT8 MFMA, TFLOP/s (TOP/s)
PEAK_HBM = 8000.0       # MI355X HBM3E, GB/s
# HBM bytes per launch of the attention kernel, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes over `python3 bench.py --probe`, each scaled by the same
# counter's reading for a device copy of known size (probe's calibration copy);
# the summary with the commands and raw readings is
# profiles/attn_bf16_pipe_s32400_h40_traffic.md: fetched 2.0 x 1718725 KiB +
# written 1.0 x 324048 KiB per launch.
TRAFFIC = 3.852e9


def attention_flops(seq, heads, dim=DIM, density=1.0):
    return 4.0 * seq * seq * heads * dim * density


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Workload:
    """Q, K, V resident on the GPU for one attention configuration."""

    def __init__(self, gpu, seq, heads, seed, scale, rope, k_bias=False):
        from h3cli_amd import synth
        lib = gpu.lib
        n = seq * heads * DIM
        self.gpu, self.seq, self.heads, self.n = gpu, seq, heads, n
        self.q, self.k, self.v = gpu.empty(n), gpu.empty(n), gpu.empty(n)
        self.out = gpu.empty(n)
        gpu.begin()
        for i, t in enumerate((self.q, self.k, self.v)):
            gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, t.handle, seed * 16 + i, scale, n), "fill")
        gpu.submit()
        if rope or k_bias:
            # Host-side preparation (outside any timed region): RoPE on Q and K,
            # or the +4.0 bias on 1% of K's channels.
            q = synth.bf16_to_f32(self.q.read()).reshape(seq, heads, DIM)
            k = synth.bf16_to_f32(self.k.read()).reshape(seq, heads, DIM)
            if rope:
                cos, sin = synth.rope_tables(*ROPE_SHAPE)
                q = synth.apply_rope(q, cos[:seq], sin[:seq])
                k = synth.apply_rope(k, cos[:seq], sin[:seq])
            if k_bias:
                rng = np.random.default_rng(seed)
                for h in range(heads):
                    k[:, h, rng.choice(DIM, size=max(1, round(0.01 * DIM)), replace=False)] += 4.0
            for t, a in ((self.q, q), (self.k, k)):
                b = synth.f32_to_bf16(a.reshape(-1))
                gpu.check(lib.h3_gpu_tensor_write_bf16(t.handle, b.ctypes.data, n), "upload")

    def call(self):
        g = self.gpu
        return g.lib.h3_gpu_dit_sdpa_bf16(g.handle, self.out.handle, self.q.handle, self.k.handle, self.v.handle,
                                          self.seq, self.heads, DIM, 1.0 / math.sqrt(DIM), 0, 0, 0)

    def host_inputs(self):
        from h3cli_amd import synth
        return [synth.bf16_to_f32(t.read()) for t in (self.q, self.k, self.v)]


def time_calls(gpu, call, steps, warmup, kernel_times=None):
    """Average ms per call between HIP events on the compute stream around the
    timed calls. With kernel_times (a list), the library also times the dominant
    kernel of every call on that stream and (avg ms, launches) is appended."""
    import ctypes as C
    gpu.begin()
    for _ in range(warmup):
        gpu.check(call(), "warmup")
    gpu.submit()
    e0, e1 = gpu.timing_event(), gpu.timing_event()
    if kernel_times is not None:
        gpu.check(gpu.lib.h3_hip_kernel_timing(gpu.handle, 1), "kernel timing")
    gpu.begin()
    gpu.record(e0)
    for _ in range(steps):
        gpu.check(call(), "timed call")
    gpu.record(e1)
    t0 = time.perf_counter()
    gpu.submit()
    wall = time.perf_counter() - t0
    ms = gpu.elapsed_ms(e0, e1)
    gpu.lib.h3_gpu_event_free(e0)
    gpu.lib.h3_gpu_event_free(e1)
    if kernel_times is not None:
        total, n = C.c_double(), C.c_uint64()
        gpu.check(gpu.lib.h3_hip_kernel_timing_read(gpu.handle, C.byref(total), C.byref(n)), "kernel timing read")
        gpu.check(gpu.lib.h3_hip_kernel_timing(gpu.handle, 0), "kernel timing")
        kernel_times.append((total.value / max(n.value, 1), n.value))
    return ms / steps, wall


def cpu_baseline(q, k, v, seq, heads, rows):
    """The oracle's online-softmax attention (reference cuda_attention.cuh:7-51
    restated in C, OpenMP over the host cores) timed twice:
    - BASELINE config 1 in full (B=1, H=8, S=1024, D=128, FP16 N(0,1) from
      seed 0, 64-key tiles): 4.295 GFLOP, measured;
    - config 2 (this bench's workload) on rows [0, rows) x all keys x all
      heads, scaled to the whole call by its row fraction: extrapolated.
    value is the config-2 rate (the metric's workload)."""
    from oracle import oracle
    scale = 1.0 / math.sqrt(DIM)
    rng = np.random.default_rng(0)
    c1 = [rng.standard_normal((1024, 8, DIM)).astype(np.float16).astype(np.float32) for _ in range(3)]
    oracle.attention(*c1, 1024, 8, scale, tile=64, rows=(0, 8))      # warm the library and page in
    t0 = time.perf_counter()
    oracle.attention(*c1, 1024, 8, scale, tile=64)
    c1_s = time.perf_counter() - t0
    c1_flops = attention_flops(1024, 8)
    t0 = time.perf_counter()
    oracle.attention(q, k, v, seq, heads, scale, tile=64, rows=(0, rows))
    dt = time.perf_counter() - t0
    flops = attention_flops(seq, heads) * rows / seq
    full_s = dt * seq / rows
    return dict(value=round(flops / dt / 1e12, 6), unit="TFLOP/s", cores=oracle.threads(), kind="port",
                sample=f"extrapolated: oracle_attention rows 0..{rows} of {seq} x {heads} heads x all keys took "
                       f"{dt:.2f} s, so a whole config-2 call takes about {full_s:.0f} s on these cores",
                extrapolated_s_per_call=round(full_s, 1),
                config1={"workload": "BASELINE config 1: B=1 H=8 S=1024 D=128 FP16 N(0,1) seed 0, full",
                         "seconds": round(c1_s, 4), "gflop": round(c1_flops / 1e9, 3),
                         "tflops": round(c1_flops / c1_s / 1e12, 6), "measured": True})


def subblock_leg(steps, warmup, sparsity=0.75):
    """Attention mode 4 with the router: a 64-row-block layout bound for S,
    sparsity 0.75 (keep = 8 * ceil(0.25 * B / 8) key blocks per query block),
    a step past the warmup and a non-probe block, so every call routes. Per
    call: pooling, block scores, selection and list build, V transpose and the
    routed attention kernel (timed on its own)."""
    import ctypes as C
    from h3cli_amd._lib import GpuStats, SolBlock, SolLayout
    from h3cli_amd.runtime import Gpu
    with Gpu() as gpu:
        lib = gpu.lib
        gpu.check(lib.h3_gpu_dit_attention_configure(gpu.handle, 4), "configure subblock")
        gpu.check(lib.h3_hip_dit_subblock_policy(gpu.handle, sparsity, 0), "policy")
        blocks = (SEQ + 63) // 64
        meta = (SolBlock * blocks)()
        for b in range(blocks):
            meta[b].rows = min(64, SEQ - b * 64)
        layout = SolLayout(SEQ, blocks, blocks, 0, C.cast(meta, C.POINTER(SolBlock)), C.cast(meta, C.POINTER(SolBlock)))
        gpu.check(lib.h3_gpu_dit_sol_layout(gpu.handle, C.byref(layout)), "layout")
        gpu.check(lib.h3_gpu_dit_attention_noise(gpu.handle, 12, 0.5, 0.5), "noise")
        log("[bench] subblock attention: preparing inputs")
        w = Workload(gpu, SEQ, HEADS, seed=2, scale=0.5, rope=True)

        def call():
            return lib.h3_gpu_dit_sdpa_bf16(gpu.handle, w.out.handle, w.q.handle, w.k.handle, w.v.handle, SEQ, HEADS,
                                            DIM, 1.0 / math.sqrt(DIM), 0, 1, 12)
        kt = []
        ms, _ = time_calls(gpu, call, steps, warmup, kt)
        st = GpuStats()
        gpu.check(lib.h3_gpu_get_stats(gpu.handle, C.byref(st)), "stats")
        density = st.subblock_selected / max(st.subblock_possible, 1)
        kernel_ms = kt[0][0]
        dense_eq = attention_flops(SEQ, HEADS) / (ms * 1e-3) / 1e12
        routed = attention_flops(SEQ, HEADS, density=density) / (kernel_ms * 1e-3) / 1e12
        log(f"[bench] subblock: {ms:.3f} ms/call, density {density:.4f}, routed kernel {kernel_ms:.3f} ms "
            f"({routed:.1f} TFLOP/s on kept tiles), router + transpose {ms - kernel_ms:.3f} ms")
        return {"workload": "SubBlock routed attention, S=32400 H=40, sparsity 0.75, no protected blocks",
                "ms_per_call": round(ms, 4), "density": round(density, 5),
                "dense_equivalent_tflops": round(dense_eq, 3), "kernel_ms": round(kernel_ms, 4),
                "kernel_tflops_on_kept_tiles": round(routed, 3),
                "kernel_frac_of_bf16_peak": round(routed / PEAK_BF16, 4),
                "router_and_transpose_ms": round(ms - kernel_ms, 4)}


def sol_leg(steps, warmup):
    """SOL routed attention (mode 3) at S = 32400, H = 40 with the reference's
    default options (tau 1, local radius 1, min-exact 0) and a layout built as
    h3_sol_layout_build does for one video segment (src/denoise/sol.c:10-58):
    27 frames of 1200 rows, first and last frames protected. Per call:
    centroids, moments, routing and lists, V transpose and the listed kernel
    (timed on its own)."""
    import ctypes as C
    from h3cli_amd._lib import SolBlock, SolLayout
    from h3cli_amd.runtime import Gpu

    class Opts(C.Structure):
        _fields_ = [("q_block", C.c_int), ("kv_block", C.c_int), ("dense_layers", C.c_int),
                    ("dense_steps", C.c_int), ("local_radius", C.c_int), ("tau", C.c_float),
                    ("min_exact", C.c_float), ("dense_sigma", C.c_float)]

    frame_rows, frames = 1200, SEQ // 1200
    out = {"workload": "SOL routed attention, S=32400 H=40, tau 1, radius 1, frames 0 and 26 protected"}
    for qblock in (32, 64):
        with Gpu() as gpu:
            lib = gpu.lib
            lib.h3_cuda_sol_exchange.restype = Opts
            lib.h3_cuda_sol_exchange.argtypes = [Opts]
            saved = lib.h3_cuda_sol_exchange(Opts(qblock, 64, 1, 1, 1, 1.0, 0.0, -1.0))
            try:
                gpu.check(lib.h3_gpu_dit_attention_configure(gpu.handle, 3), "configure sol")
            finally:
                lib.h3_cuda_sol_exchange(saved)
            arrays = []
            for block in (qblock, 64):
                nb = (SEQ + block - 1) // block
                arr = (SolBlock * nb)()
                for b in range(nb):
                    r0, r1 = b * block, min(SEQ, b * block + block) - 1
                    f0, f1 = r0 // frame_rows, r1 // frame_rows
                    arr[b].rows = r1 - r0 + 1
                    arr[b].first_frame, arr[b].last_frame = f0, f1
                    arr[b].protect = int(f0 == 0 or f1 == frames - 1)
                arrays.append(arr)
            layout = SolLayout(SEQ, len(arrays[0]), len(arrays[1]), 0, C.cast(arrays[0], C.POINTER(SolBlock)),
                               C.cast(arrays[1], C.POINTER(SolBlock)))
            gpu.check(lib.h3_gpu_dit_sol_layout(gpu.handle, C.byref(layout)), "layout")
            gpu.check(lib.h3_gpu_dit_attention_noise(gpu.handle, 5, 0.2, 0.2), "noise")
            w = Workload(gpu, SEQ, HEADS, seed=2, scale=0.5, rope=True)

            def call():
                return lib.h3_gpu_dit_sdpa_bf16(gpu.handle, w.out.handle, w.q.handle, w.k.handle, w.v.handle, SEQ,
                                                HEADS, DIM, 1.0 / math.sqrt(DIM), 0, 1, 5)
            kt = []
            ms, _ = time_calls(gpu, call, steps, warmup, kt)
            QB, KB = (SEQ + qblock - 1) // qblock, (SEQ + 63) // 64
            routes = np.zeros(HEADS * QB * KB, np.uint8)
            gpu.check(lib.h3_hip_sol_routes(gpu.handle, routes.ctypes.data, routes.size, None, 0, None, None, 0),
                      "routes")
            density = float(routes.mean())
        kernel_ms = kt[0][0]
        tf = attention_flops(SEQ, HEADS, density=density) / (kernel_ms * 1e-3) / 1e12
        log(f"[bench] sol q{qblock}: {ms:.3f} ms/call, exact density {density:.4f}, listed kernel {kernel_ms:.3f} ms "
            f"({tf:.1f} TFLOP/s on exact tiles), routing + transpose {ms - kernel_ms:.3f} ms")
        out[f"q{qblock}"] = {"ms_per_call": round(ms, 4), "exact_density": round(density, 5),
                             "kernel_ms": round(kernel_ms, 4), "kernel_tflops_on_exact_tiles": round(tf, 2),
                             "routing_and_transpose_ms": round(ms - kernel_ms, 4)}
    return out


GEMM_SHAPES = [("qkv", 5120, 15360, False), ("out", 5120, 5120, False), ("up_gelu", 5120, 13824, True),
               ("down", 13824, 5120, False)]


def gemm_leg(steps, warmup, m=32400, seed=4):
    """W8A16 GEMMs of one DiT block at M = 32400 rows, int8
    weights U[-127,127] with per-output-channel fp32 scales U[1e-3,1e-2]."""
    from h3cli_amd.runtime import Gpu, Tensor
    out = {"workload": "W8A16 GEMM set of one DiT block (BASELINE config 4)", "rows": m, "shapes": {}}
    total_flops, total_ms = 0.0, 0.0
    with Gpu() as gpu:
        lib = gpu.lib
        x = gpu.empty(m * 13824)
        gpu.begin()
        gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, x.handle, seed * 16, 1.0, m * 13824), "fill")
        gpu.submit()
        rng = np.random.default_rng(seed)
        for name, k, n, gelu in GEMM_SHAPES:
            codes = rng.integers(-127, 128, size=n * k, dtype=np.int8)
            scales = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
            h = lib.h3_hip_q8_from_packed(gpu.handle, codes.ctypes.data, scales.ctypes.data, n, k, k)
            if not h:
                raise RuntimeError(gpu.error())
            w = Tensor(gpu, h, n * k, 2)
            gpu.tensors.append(w)
            y = gpu.empty(m * n)
            fn = lib.h3_hip_linear_gelu_bf16 if gelu else lib.h3_gpu_linear_bf16
            call = lambda: fn(gpu.handle, y.handle, x.handle, w.handle, None, m, k, n)
            kt = []
            ms, _ = time_calls(gpu, call, steps, warmup, kt)
            flops = 2.0 * m * k * n
            total_flops += flops
            total_ms += ms
            out["shapes"][name] = {"k": k, "n": n, "ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2),
                                   "kernel_ms": round(kt[0][0], 4)}
            log(f"[bench] gemm {name} {m}x{k}x{n}: {ms:.3f} ms, {flops / ms / 1e9:.1f} TFLOP/s")
            gpu.free(y)
            gpu.free(w)
    out["ms_total"] = round(total_ms, 4)
    out["tflops"] = round(total_flops / total_ms / 1e9, 2)
    out["frac_of_bf16_peak"] = round(total_flops / total_ms / 1e9 / PEAK_BF16, 4)
    return out


def _time_steps(steps, warmup, **overrides):
    from h3cli_amd.runtime import DitSynth
    t0 = time.perf_counter()
    with DitSynth(**overrides) as m:
        setup = time.perf_counter() - t0
        kept, total = m.kept_blocks()
        rows, cfg = m.rows, m.config
        for i in range(warmup):
            m.step(step=i, dt=-0.02)
        times = []
        for i in range(steps):
            t1 = time.perf_counter()
            m.step(step=warmup + i, dt=-0.02)
            times.append(time.perf_counter() - t1)
        finite = bool(np.all(np.isfinite(m.read("latent"))))
    return float(np.mean(times)), setup, kept, total, rows, cfg, finite


def step_leg(steps, warmup):
    """one full 40-block synthetic DiT denoise step (M = 32400
    video + 1024 audio rows, hidden 5120, 40 heads, MLP 13824, W8A16 weights,
    Sage attention over a 25%-density 128x128 block mask plus audio<->audio and
    the diagonal, blocks 20-39 streamed from pinned host memory). The same step
    with every block resident is timed beside it: the difference is what the
    4.93 GB of host-to-device weight copies per step cost beyond compute."""
    sec, setup, kept, total, rows, cfg, finite = _time_steps(steps, warmup)
    resident, _, _, _, _, _, finite_r = _time_steps(steps, warmup, streamed_first=40)
    H = cfg.hidden
    gemm = 2.0 * rows * (H * 3 * H + H * H + 2 * H * cfg.mlp) * cfg.blocks
    head = 2.0 * rows * cfg.latent * H * 2
    density = kept / total
    attn = attention_flops(rows, cfg.heads) * density * cfg.blocks
    streamed_blocks = cfg.blocks - cfg.streamed_first
    log(f"[bench] full step: {sec:.3f} s/step streamed, {resident:.3f} s/step resident (setup {setup:.1f} s), "
        f"mask density {density:.4f}, finite={finite and finite_r}")
    return {"workload": "full synthetic 40-block DiT denoise step (BASELINE config 5)",
            "s_per_step": round(sec, 4), "s_per_step_all_resident": round(resident, 4),
            "streaming_overhead": round(sec / resident - 1, 4), "steps": steps, "warmup": warmup, "rows": rows,
            "blocks": cfg.blocks, "streamed_blocks": streamed_blocks,
            "streamed_bytes_per_step": streamed_blocks * (
                H * 3 * H + H * H + 2 * H * cfg.mlp + 4 * (3 * H + H + cfg.mlp + H)),
            "mask_kept_blocks": kept, "mask_total_blocks": total, "mask_density": round(density, 5),
            "gemm_tflop": round(gemm / 1e12, 3), "attention_tflop_effective": round(attn / 1e12, 3),
            "achieved_tflops": round((gemm + head + attn) / sec / 1e12, 2), "latent_finite": finite and finite_r,
            "setup_s": round(setup, 1)}


# The reference's published real-H3 figures (other hardware), for the legs below.
H3_PUBLISHED = {
    "attention_18225": {"cudnn_bf16_ms": {"RTX 5090": 40.419, "RTX PRO 6000": 24.291, "H100": 14.347, "B200": 6.270},
                        "sage2pp_ms": {"RTX 5090": 19.056},
                        "source": "docs/cuda/attention-validation.md:54, cuda-fast-validation.md:13,120, "
                                  "cuda-h100-qualification.md:90, cuda-b200-qualification.md:122"},
    "attention_109078": {"cudnn_bf16_ms": {"RTX 5090": 1485.910}, "sage2pp_ms": {"RTX 5090": 609.853},
                         "source": "docs/cuda/attention-validation.md:56"},
    "proj_8193": {"bf16_ms": {"RTX 5090": 26.415}, "fp8_ms": {"RTX 5090": 15.767}, "nvfp4_ms": {"RTX 5090": 7.281},
                  "source": "docs/cuda/denoiser-quantization-validation.md:174-177"},
}


def h3_attention_leg(seqs=(18225, 109078), heads=56):
    """Real-H3 attention (H = 56, D = 128) at the reference's published token
    counts: dense BF16 and Sage2++ (int8 QK / fp8 PV, quantization included)
    per call, on seeded 0.5 N(0,1) Q/K/V resident in HBM."""
    from h3cli_amd.runtime import Gpu
    out = {"workload": "real-H3 attention, H=56 D=128, per call", "published": {}}
    for seq in seqs:
        steps, warmup = (5, 1) if seq < 50000 else (2, 1)
        row = {}
        for name, mode in (("bf16", 0), ("sage2pp", 1)):
            with Gpu() as gpu:
                gpu.check(gpu.lib.h3_gpu_dit_attention_configure(gpu.handle, mode), "configure")
                w = Workload(gpu, seq, heads, seed=7, scale=0.5, rope=False)
                ms, _ = time_calls(gpu, w.call, steps, warmup)
            tf = attention_flops(seq, heads) / (ms * 1e-3) / 1e12
            row[name] = {"ms": round(ms, 3), "tflops": round(tf, 1)}
            log(f"[bench] h3 attention S={seq} H={heads} {name}: {ms:.3f} ms ({tf:.1f} TFLOP/s)")
        out[f"s{seq}"] = row
        out["published"][f"s{seq}"] = H3_PUBLISHED[f"attention_{seq}"]
    return out


def h3_proj_leg(steps, warmup, m=8193, seed=9):
    """The four real-H3 block projections at 8,193 rows (reference
    quant_prepare.c:20 shapes): qkv 5376 -> 21504, out 7168 -> 5376, fc1 5376 ->
    28672, fc2 14336 -> 5376, as W8A16 in the reference q8 recipe (int8 codes,
    fp32 scale per 64 columns) with BF16 activations."""
    from h3cli_amd.runtime import Gpu, Tensor
    shapes = [("qkv", 5376, 21504), ("out", 7168, 5376), ("fc1", 5376, 28672), ("fc2", 14336, 5376)]
    res = {"workload": "real-H3 block-0 projections, 8193 rows, W8A16 (q8 group 64)", "rows": m, "shapes": {},
           "published": H3_PUBLISHED["proj_8193"]}
    total_flops, total_ms = 0.0, 0.0
    with Gpu() as gpu:
        lib = gpu.lib
        x = gpu.empty(m * 14336)
        gpu.begin()
        gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, x.handle, seed * 16, 1.0, m * 14336), "fill")
        gpu.submit()
        for i, (name, k, n) in enumerate(shapes):
            w = Tensor(gpu, lib.h3_hip_q8_new(gpu.handle, n, k, 64), n * k, 2)
            gpu.tensors.append(w)
            gpu.begin()
            gpu.check(lib.h3_hip_fill_q8_random(gpu.handle, w.handle, seed * 8 + i, C_float(1e-3), C_float(1e-2)),
                      "fill q8")
            gpu.submit()
            y = gpu.empty(m * n)
            call = lambda: lib.h3_gpu_linear_bf16(gpu.handle, y.handle, x.handle, w.handle, None, m, k, n)
            ms, _ = time_calls(gpu, call, steps, warmup)
            flops = 2.0 * m * k * n
            total_flops += flops
            total_ms += ms
            res["shapes"][name] = {"k": k, "n": n, "ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2)}
            log(f"[bench] h3 proj {name} {m}x{k}x{n}: {ms:.3f} ms, {flops / ms / 1e9:.1f} TFLOP/s")
            gpu.free(y)
            gpu.free(w)
    res["ms_total"] = round(total_ms, 4)
    res["tflops"] = round(total_flops / total_ms / 1e9, 2)
    return res


def h3_proj_quant_leg(steps, warmup, mode=1, m=8193, seed=9):
    """The same four real-H3 projections quantized (reference
    cuda_quant.cuh:339-398, the modes behind the published FP8 and NVFP4
    figures). mode 1, FP8 W8A8: tensorwide E4M3 weights packed once, the
    activation packed per call (max, scale, encode), then the FP8 GEMM. mode 2,
    NVFP4 W4A4: weights packed and dequantized to BF16 once, the activation
    packed and dequantized per call, then the BF16 GEMM with alpha. ms is the
    whole call; gemm_ms the GEMM kernel."""
    from h3cli_amd.runtime import Gpu, Tensor
    shapes = [("qkv", 5376, 21504), ("out", 7168, 5376), ("fc1", 5376, 28672), ("fc2", 14336, 5376)]
    kind = "FP8 W8A8 (tensorwide E4M3)" if mode == 1 else "NVFP4 W4A4 (UE4M3 per 16, dequantized to BF16)"
    res = {"workload": f"real-H3 block-0 projections, 8193 rows, {kind}", "rows": m, "shapes": {},
           "published": H3_PUBLISHED["proj_8193"]}
    total_flops, total_ms, total_gemm = 0.0, 0.0, 0.0
    with Gpu() as gpu:
        lib = gpu.lib
        gpu.check(lib.h3_gpu_quant_configure(gpu.handle, mode, os.environ.get("TMPDIR", "/tmp").encode() + b"/h3-quant",
                                             2 * (4 * 7168 * 5376 + 3 * 14336 * 5376), 1 << 30, 0), "quant configure")
        x = gpu.empty(m * 14336)
        gpu.begin()
        gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, x.handle, seed * 16, 1.0, m * 14336), "fill")
        gpu.submit()
        for i, (name, k, n) in enumerate(shapes):
            wb = gpu.empty(n * k)
            gpu.begin()
            gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, wb.handle, seed * 8 + i, 0.02, n * k), "fill w")
            gpu.submit()
            h = lib.h3_hip_quant_weight_from_bf16(gpu.handle, wb.handle, n, k)
            gpu.check(h, "quantized weight")
            w = Tensor(gpu, h, n * k, 2)
            gpu.tensors.append(w)
            gpu.free(wb)
            y = gpu.empty(m * n)
            call = lambda: lib.h3_gpu_linear_bf16(gpu.handle, y.handle, x.handle, w.handle, None, m, k, n)
            kt = []
            ms, _ = time_calls(gpu, call, steps, warmup, kt)
            flops = 2.0 * m * k * n
            total_flops += flops
            total_ms += ms
            total_gemm += kt[0][0]
            res["shapes"][name] = {"k": k, "n": n, "ms": round(ms, 4), "gemm_ms": round(kt[0][0], 4),
                                   "tflops": round(flops / ms / 1e9, 2), "gemm_tflops": round(flops / kt[0][0] / 1e9, 2)}
            log(f"[bench] h3 {'fp8' if mode == 1 else 'nvfp4'} proj {name} {m}x{k}x{n}: {ms:.3f} ms per call, GEMM {kt[0][0]:.3f} ms "
                f"({flops / kt[0][0] / 1e9:.1f} TFLOP/s)")
            gpu.free(y)
            gpu.free(w)
    res["ms_total"] = round(total_ms, 4)
    res["gemm_ms_total"] = round(total_gemm, 4)
    res["tflops"] = round(total_flops / total_ms / 1e9, 2)
    return res


def h3_step_leg(steps, warmup, fp8=False):
    """One real-H3-geometry denoise step (include/h3_dit_synth.h
    h3_hip_dit_synth_h3): 50 blocks, 18225 video rows, hidden 5376, 56 heads,
    grouped QKV with Q/K norm, 48 RoPE pairs, SwiGLU 14336, all weights
    resident, dense BF16 attention; projections W8A16, or FP8 W8A8 (tensorwide
    E4M3, activations packed per call) with fp8."""
    from h3cli_amd.runtime import DitSynth
    t0 = time.perf_counter()
    with DitSynth(geometry="h3", projection_quant=1 if fp8 else 0) as m:
        setup = time.perf_counter() - t0
        rows, cfg = m.rows, m.config
        for i in range(warmup):
            m.step(step=i, dt=-0.02)
        times = []
        for i in range(steps):
            t1 = time.perf_counter()
            m.step(step=warmup + i, dt=-0.02)
            times.append(time.perf_counter() - t1)
        finite = bool(np.all(np.isfinite(m.read("latent"))))
    sec = float(np.mean(times))
    H, I, F = cfg.hidden, cfg.heads * 128, cfg.mlp
    gemm = 2.0 * rows * (H * 3 * I + I * H + H * 2 * F + F * H) * cfg.blocks
    attn = attention_flops(rows, cfg.heads) * cfg.blocks
    kind = "FP8 W8A8" if fp8 else "W8A16"
    log(f"[bench] h3 step ({kind}): {sec:.3f} s/step over {rows} rows (setup {setup:.1f} s), finite={finite}")
    return {"workload": f"real-H3-geometry 50-block denoise step, 18225 rows, dense BF16 attention, {kind} projections",
            "s_per_step": round(sec, 4), "steps": steps, "rows": rows, "blocks": cfg.blocks,
            "gemm_tflop": round(gemm / 1e12, 3), "attention_tflop": round(attn / 1e12, 3),
            "achieved_tflops": round((gemm + attn) / sec / 1e12, 2), "latent_finite": finite,
            "setup_s": round(setup, 1)}


def probe(scale=0.5):
    """Launches for HBM-traffic counters: attention twice (config 2 inputs),
    then a plain device-to-device copy of exactly 2^30 bytes, whose FETCH_SIZE
    and WRITE_SIZE readings calibrate the counters (2^30 bytes each way).
    scale multiplies the N(0,1) inputs; 0 gives all-zero operands (for the
    clock the same kernel reaches at a lower power draw)."""
    from h3cli_amd.runtime import Gpu
    with Gpu() as gpu:
        w = Workload(gpu, SEQ, HEADS, seed=2, scale=scale, rope=False)
        gpu.begin()
        for _ in range(2):
            gpu.check(w.call(), "attention")
        gpu.submit()
        n = (1 << 30) // 2
        src, dst = gpu.empty(n), gpu.empty(n)
        gpu.begin()
        gpu.check(gpu.lib.h3_hip_fill_normal_bf16(gpu.handle, src.handle, 7, 1.0, n), "fill copy source")
        gpu.check(gpu.lib.h3_hip_fill_normal_bf16(gpu.handle, dst.handle, 8, 1.0, n), "fill copy target")
        gpu.submit()
        gpu.begin()
        gpu.check(gpu.lib.h3_gpu_copy_bf16(gpu.handle, dst.handle, 0, src.handle, 0, n), "copy")
        gpu.submit()
    log("[probe] 2 attention launches (S=32400, H=40) + 1 GiB device copy done")


def probe_sage(scale=1.0):
    """Two Sage attention calls on config 3's inputs (N(0,1) times scale, the
    +4.0 channel bias when scale > 0), for counters; nothing timed. scale 0
    gives all-zero int8 and fp8 operands."""
    from h3cli_amd.runtime import Gpu
    with Gpu() as gpu:
        gpu.check(gpu.lib.h3_gpu_dit_attention_configure(gpu.handle, 1), "configure sage2++")
        w = Workload(gpu, SEQ, HEADS, seed=3, scale=scale, rope=False, k_bias=scale > 0)
        gpu.begin()
        for _ in range(2):
            gpu.check(w.call(), "sage attention")
        gpu.submit()
    log(f"[probe-sage] 2 Sage attention calls (S={SEQ}, H={HEADS}, input scale {scale})")


def probe_gemm(which, m=32400, k=5120, n=15360, x_scale=1.0):
    """Launches for SQ counters on config 4's QKV shape, nothing timed: this
    library's W8A16 projection twice (dequantization + GEMM), or, as the
    calibration point, hipBLASLt's BF16 GEMM (torch.matmul on BF16 weights of
    the same shape) twice. The hipBLASLt probe never loads this library (two
    HIP runtimes in one process do not share the device). x_scale multiplies
    this library's N(0,1) activations (0: all-zero X)."""
    if which == "hipblaslt":
        import torch
        x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        w = torch.randn(n, k, device="cuda", dtype=torch.bfloat16) * 0.02
        for _ in range(2):
            y = torch.matmul(x, w.t())
        torch.cuda.synchronize()
        log(f"[probe-gemm] hipBLASLt BF16 {m}x{k}x{n} twice, finite={bool(torch.isfinite(y).all())}")
        return
    from h3cli_amd.runtime import Gpu, Tensor
    with Gpu() as gpu:
        lib = gpu.lib
        x = gpu.empty(m * k)
        gpu.begin()
        gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, x.handle, 64, x_scale, m * k), "fill")
        gpu.submit()
        rng = np.random.default_rng(4)
        codes = rng.integers(-127, 128, size=n * k, dtype=np.int8)
        scales = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
        h = lib.h3_hip_q8_from_packed(gpu.handle, codes.ctypes.data, scales.ctypes.data, n, k, k)
        if not h:
            raise RuntimeError(gpu.error())
        w = Tensor(gpu, h, n * k, 2)
        gpu.tensors.append(w)
        y = gpu.empty(m * n)
        gpu.begin()
        for _ in range(2):
            gpu.check(lib.h3_gpu_linear_bf16(gpu.handle, y.handle, x.handle, w.handle, None, m, k, n), "W8A16 GEMM")
        gpu.submit()
    log(f"[probe-gemm] W8A16 {m}x{k}x{n} twice")


def profile_step():
    """One warmup and one timed config-5 step (blocks 20-39 streamed), nothing
    else: the program to run under `rocprofv3 --kernel-trace
    --memory-copy-trace` to see the weight copies beside the kernels."""
    from h3cli_amd.runtime import DitSynth
    with DitSynth() as m:
        m.step(step=0, dt=-0.02)
        t0 = time.perf_counter()
        m.step(step=1, dt=-0.02)
        log(f"[profile-step] one streamed config-5 step: {time.perf_counter() - t0:.3f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--legs", default="attention,sage,subblock,sol,gemm,step,h3_attention,h3_proj,h3_proj_fp8,h3_proj_nvfp4,h3_step,h3_step_fp8")
    ap.add_argument("--step-count", type=int, default=3, help="timed full DiT steps (step leg)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=int(os.environ.get("H3_BENCH_CPU_ROWS", "576")))
    ap.add_argument("--probe", action="store_true",
                    help="counter probe for rocprofv3 --pmc: two attention launches and one 1 GiB device copy "
                         "(the calibration kernel), nothing timed")
    ap.add_argument("--probe-sage", action="store_true",
                    help="counter probe: two Sage attention calls on config 3's inputs")
    ap.add_argument("--probe-scale", type=float, default=None,
                    help="with --probe, --probe-sage or --probe-gemm h3: scale of the N(0,1) inputs (0: all-zero operands)")
    ap.add_argument("--probe-gemm", choices=["h3", "hipblaslt"],
                    help="counter probe: config 4's QKV projection twice, this library's or hipBLASLt's BF16 GEMM")
    ap.add_argument("--profile-step", action="store_true",
                    help="two config-5 steps with streamed weights and nothing else, for a rocprofv3 trace")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the DiT hot path here runs on a single MI355X "
              "(multi-GPU sharding is a design note, not part of this build).", file=sys.stderr)
        sys.exit(2)

    if args.probe_gemm:
        probe_gemm(args.probe_gemm, x_scale=1.0 if args.probe_scale is None else args.probe_scale)
        return
    from h3cli_amd.runtime import Gpu
    if args.probe:
        probe(0.5 if args.probe_scale is None else args.probe_scale)
        return
    if args.probe_sage:
        probe_sage(1.0 if args.probe_scale is None else args.probe_scale)
        return
    if args.profile_step:
        profile_step()
        return
    legs = [x for x in args.legs.split(",") if x]
    result = {}
    with Gpu() as gpu:
        log(f"[bench] bf16 attention S={SEQ} H={HEADS}: preparing inputs")
        w = Workload(gpu, SEQ, HEADS, seed=2, scale=0.5, rope=True)
        kt = []
        ms, wall = time_calls(gpu, w.call, args.steps, args.warmup, kt)
        flops = attention_flops(SEQ, HEADS)
        tflops = flops / (ms * 1e-3) / 1e12
        kernel_ms, kernel_n = kt[0]
        kernel_tflops = flops / (kernel_ms * 1e-3) / 1e12
        log(f"[bench] bf16 attention: {ms:.3f} ms/call, {tflops:.1f} TFLOP/s; "
            f"attention kernel {kernel_ms:.3f} ms avg over {kernel_n} launches ({kernel_tflops:.1f} TFLOP/s)")
        result.update({
            "metric": "attention TFLOP/s + %MFMA peak; s/denoise-step (40-block DiT, S=32400) 1 GPU",
            "value": round(tflops, 3),
            "unit": "TFLOP/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms, 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic: seeded 0.5*N(0,1) bf16 Q/K/V with 3D RoPE (44/42/42, theta 1e4) on Q,K",
            "config": {"workload": "bf16 DiT video self-attention (BASELINE config 2)", "seq": SEQ,
                       "heads": HEADS, "head_dim": DIM, "batch": 1, "flop_convention": "4*S^2*H*D"},
            "roofline": {"bound": "mfma", "achieved": round(kernel_tflops, 3), "peak": PEAK_BF16,
                         "unit": "TFLOP/s", "frac": round(kernel_tflops / PEAK_BF16, 4), "traffic": TRAFFIC,
                         "kernel": "attn_bf16_pipe + recomputation launch", "kernel_ms": round(kernel_ms, 4),
                         "kernel_launches": kernel_n, "traffic_unit": "HBM bytes per launch (rocprofv3, calibrated)",
                         "algorithmic": "4*S^2*H*D = 21.499 TFLOP per launch (one launch covers all 40 heads)"},
        })
        if not args.no_cpu:
            log(f"[bench] CPU baseline on {args.cpu_rows} rows")
            q, k, v = w.host_inputs()
            result["cpu_baseline"] = cpu_baseline(q, k, v, SEQ, HEADS, args.cpu_rows)
            del q, k, v
        for t in (w.q, w.k, w.v, w.out):
            gpu.free(t)

    if "sage" in legs:
        with Gpu() as gpu:
            gpu.check(gpu.lib.h3_gpu_dit_attention_configure(gpu.handle, 1), "configure sage2++")
            log("[bench] sage attention: preparing inputs")
            w = Workload(gpu, SEQ, HEADS, seed=3, scale=1.0, rope=False, k_bias=True)
            kt = []
            ms_s, _ = time_calls(gpu, w.call, args.steps, args.warmup, kt)
            eff = attention_flops(SEQ, HEADS) / (ms_s * 1e-3) / 1e12
            log(f"[bench] sage attention: {ms_s:.3f} ms/call, {eff:.1f} effective TFLOP/s; "
                f"attention kernel {kt[0][0]:.3f} ms (quantizers {ms_s - kt[0][0]:.3f} ms)")
            result["sage"] = {"workload": "Sage int8-QK / fp8-PV attention (BASELINE config 3), incl. quantization",
                              "ms_per_call": round(ms_s, 4), "effective_tflops": round(eff, 3),
                              "speedup_vs_bf16": round(ms / ms_s, 3),
                              "kernel_ms": round(kt[0][0], 4),
                              "frac_of_fp8_peak": round(eff / PEAK_FP8, 4)}
    if "subblock" in legs:
        result["subblock"] = subblock_leg(args.steps, args.warmup)
    if "sol" in legs:
        result["sol"] = sol_leg(args.steps, args.warmup)
    if "gemm" in legs:
        result["gemm"] = gemm_leg(args.steps, args.warmup)
    if "h3_attention" in legs:
        result["h3_attention"] = h3_attention_leg()
    if "h3_proj" in legs:
        result["h3_proj"] = h3_proj_leg(args.steps, args.warmup)
    if "h3_proj_fp8" in legs:
        result["h3_proj_fp8"] = h3_proj_quant_leg(args.steps, args.warmup, mode=1)
    if "h3_proj_nvfp4" in legs:
        result["h3_proj_nvfp4"] = h3_proj_quant_leg(args.steps, args.warmup, mode=2)
    if "h3_step" in legs:
        result["h3_step"] = h3_step_leg(2, 1)
    if "h3_step_fp8" in legs:
        result["h3_step_fp8"] = h3_step_leg(2, 1, fp8=True)
    if "step" in legs:
        result["step"] = step_leg(args.step_count, 1)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
