"""Checkpoint loading into the DiT step (h3_hip_dit_synth_load): a safetensors
file with the reference's block tensor names (src/denoise/dit.c:592-611),
written by the `safetensors` package. Loaded projections must equal the
reference q8 recipe applied to the file's BF16 weights bit for bit, norms must
equal the file, the loaded model must step deterministically, and missing or
mismatched tensors must be named in the error."""
import os

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd.runtime import DitSynth, H3Error
from oracle import oracle

pytestmark = pytest.mark.gpu

SMALL = dict(blocks=2, hidden=512, heads=3, mlp=768, frames=3, height=8, width=200, latent=256, seed=4,
             streamed_first=2)


def checkpoint(path, drop=None, reshape=None, f32=None):
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(21)
    H, I, F = SMALL["hidden"], SMALL["heads"] * 128, SMALL["mlp"]
    shapes = {"norm1.weight": (H,), "norm2.weight": (H,), "attn.qkv_proj.weight": (3 * I, H),
              "attn.q_norm.weight": (128,), "attn.k_norm.weight": (128,), "attn.out_proj.weight": (H, I),
              "mlp.fc1.weight": (2 * F, H), "mlp.fc2.weight": (H, F)}
    tensors = {}
    for b in range(SMALL["blocks"]):
        for suffix, shape in shapes.items():
            scale = 0.05 if len(shape) == 2 else 0.1
            t = torch.randn(*shape, generator=g) * scale + (1.0 if len(shape) == 1 else 0.0)
            tensors[f"blocks.{b}.{suffix}"] = t.to(torch.bfloat16)
    tensors["unrelated.bias"] = torch.zeros(7, dtype=torch.bfloat16)
    if drop:
        del tensors[drop]
    if reshape:
        tensors[reshape] = tensors[reshape].reshape(-1)
    if f32:
        tensors[f32] = tensors[f32].float()
    save_file(tensors, str(path), metadata={"format": "pt"})
    return {k: v.view(torch.int16).numpy().view(np.uint16).copy() for k, v in tensors.items() if v.dtype == torch.bfloat16}


def test_load_weights_bit_exact_and_step(tmp_path):
    path = tmp_path / "h3.safetensors"
    ref = checkpoint(path)
    runs = []
    for _ in range(2):
        with DitSynth(geometry="h3", **SMALL) as m:
            m.load(path)
            for b in range(SMALL["blocks"]):
                for suffix in ("attn.qkv_proj.weight", "attn.out_proj.weight", "mlp.fc1.weight", "mlp.fc2.weight"):
                    name = f"blocks.{b}.{suffix}"
                    h = m.lib.h3_hip_dit_synth_tensor(m.handle, name.encode())
                    assert h, name
                    w = ref[name]
                    n, k = {"attn.qkv_proj.weight": (3 * 384, 512), "attn.out_proj.weight": (512, 384),
                            "mlp.fc1.weight": (1536, 512), "mlp.fc2.weight": (512, 768)}[suffix]
                    groups = (k + 63) // 64
                    raw = np.zeros(n * k + n * groups * 4, np.uint8)
                    assert m.lib.h3_hip_tensor_copy_to_host(h, raw.ctypes.data, raw.size), m.gpu.error()
                    codes, scales = oracle.q8_pack(w, n, k, 64)
                    assert np.array_equal(raw[:n * k].view(np.int8), codes), name
                    assert np.array_equal(raw[n * k:].view(np.float32), scales), name
                for suffix in ("norm1.weight", "norm2.weight", "attn.q_norm.weight", "attn.k_norm.weight"):
                    name = f"blocks.{b}.{suffix}"
                    assert np.array_equal(m.read(name), ref[name]), name
            m.step(step=0, dt=-0.1)
            runs.append((m.read("latent"), m.read("hidden")))
    assert np.all(np.isfinite(runs[0][0])) and np.all(np.isfinite(synth.bf16_to_f32(runs[0][1])))
    assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1])
    with DitSynth(geometry="h3", **SMALL) as m:
        m.step(step=0, dt=-0.1)
        assert not np.array_equal(m.read("hidden"), runs[0][1])      # the loaded weights were used


@pytest.mark.parametrize("kind,name", [("drop", "blocks.1.mlp.fc2.weight"), ("reshape", "blocks.0.attn.out_proj.weight"),
                                       ("f32", "blocks.0.norm2.weight")])
def test_load_errors_name_the_tensor(tmp_path, kind, name):
    path = tmp_path / "bad.safetensors"
    checkpoint(path, **{kind: name})
    with DitSynth(geometry="h3", **SMALL) as m:
        with pytest.raises(H3Error) as e:
            m.load(path)
        assert f"missing/invalid {name}" in str(e.value)


def test_load_needs_resident_blocks(tmp_path):
    path = tmp_path / "h3.safetensors"
    checkpoint(path)
    with DitSynth(geometry="h3", **dict(SMALL, streamed_first=1)) as m:
        with pytest.raises(H3Error) as e:
            m.load(path)
        assert "resident" in str(e.value)


@pytest.mark.parametrize("mode", [1, 2], ids=["fp8", "nvfp4"])
def test_load_quantized_projections(tmp_path, monkeypatch, mode):
    """projection_quant 1 (FP8) / 2 (NVFP4): the checkpoint's projections go
    through h3_gpu_quant_load (the artifact cache under $TMPDIR) and equal the
    reference's descriptor of the file's BF16 weights byte for byte; the step
    is deterministic and tracks the W8A16 model loaded from the same file."""
    from tests.test_quant_gpu import descriptor, nvfp4_descriptor, packed_size
    monkeypatch.setenv("TMPDIR", str(tmp_path))
    path = tmp_path / "h3.safetensors"
    ref = checkpoint(path)
    shapes = {"attn.qkv_proj.weight": (3 * 384, 512), "attn.out_proj.weight": (512, 384),
              "mlp.fc1.weight": (1536, 512), "mlp.fc2.weight": (512, 768)}
    hidden = []
    for run in range(2):
        with DitSynth(geometry="h3", projection_quant=mode, **dict(SMALL, streamed_first=SMALL["blocks"])) as m:
            m.load(path)
            if run == 0:
                for b in range(SMALL["blocks"]):
                    for suffix, (n, k) in shapes.items():
                        name = f"blocks.{b}.{suffix}"
                        h = m.lib.h3_hip_dit_synth_tensor(m.handle, name.encode())
                        want, _ = descriptor(ref[name], n, k) if mode == 1 else nvfp4_descriptor(ref[name], n, k)
                        raw = np.zeros(packed_size(n, k, mode)[2], np.uint8)
                        assert m.lib.h3_hip_tensor_copy_to_host(h, raw.ctypes.data, raw.size), m.gpu.error()
                        assert np.array_equal(raw, want), name
            m.step(step=0, dt=-0.1)
            hidden.append(m.read("hidden"))
    assert any(f.endswith(".h3q") for f in os.listdir(tmp_path / "h3cli-amd-quant"))
    assert np.array_equal(hidden[0], hidden[1]) and np.all(np.isfinite(synth.bf16_to_f32(hidden[0])))
    with DitSynth(geometry="h3", **SMALL) as m:
        m.load(path)
        m.step(step=0, dt=-0.1)
        q8 = synth.bf16_to_f32(m.read("hidden")).astype(np.float64)
    f8 = synth.bf16_to_f32(hidden[0]).astype(np.float64)
    cos = np.dot(f8, q8) / np.sqrt(np.dot(f8, f8) * np.dot(q8, q8))
    assert cos > (0.99 if mode == 1 else 0.95), cos
