"""numpy binding of oracle/_build/liboracle.so — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, as the checker or the timed CPU baseline. The product path
(h3cli_amd / libh3hip.so) never does."""
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"
_lib = None

_p = C.c_void_p
_u = C.c_uint
_f = C.c_float


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = C.CDLL(str(LIB))
        lib.oracle_attention.argtypes = [_p, _p, _p, _p, _u, _u, _u, _f, _u, _u, _u]
        lib.oracle_attention_masked.argtypes = [_p, _p, _p, _p, _u, _u, _u, _f, _p, _u, _u, _u]
        lib.oracle_attention_f64.argtypes = [_p, _p, _p, _p, _u, _u, _u, C.c_double, _u, _u]
        lib.oracle_sage_pack.argtypes = [_p, _p, _p, _u, _u, _p, _p, _p, _p, _p, _p, _p]
        lib.oracle_k_mean_f64.argtypes = [_p, _u, _u, _p]
        lib.oracle_sage_attention.argtypes = [_p, _p, _p, _p, _p, _p, _p, _u, _u, _f, _p, _u, _u, _u]
        lib.oracle_f32_to_e4m3.argtypes = [_f]
        lib.oracle_f32_to_e4m3.restype = C.c_uint8
        lib.oracle_e4m3_to_f32.argtypes = [C.c_uint8]
        lib.oracle_e4m3_to_f32.restype = _f
        lib.oracle_sage_v_position.argtypes = [_u]
        lib.oracle_sage_v_position.restype = _u
        lib.oracle_threads.restype = C.c_int
        lib.oracle_xorshift_bf16.argtypes = [_p, C.c_size_t, _p]
        lib.oracle_xorshift_native_bf16.argtypes = [_p, C.c_size_t, _p]
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data if a is not None else None


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def attention(q, k, v, seq, heads, scale, tile=64, rows=None, mask=None, block=128):
    """Online-softmax FP32 attention on float32 [seq, heads, 128] inputs; returns
    float32 [len(rows), heads, 128]."""
    lib = load()
    r0, r1 = rows if rows is not None else (0, seq)
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros((r1 - r0, heads, 128), dtype=np.float32)
    if mask is None:
        lib.oracle_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), seq, heads, 128, scale, tile, r0, r1)
    else:
        m = np.ascontiguousarray(mask, dtype=np.uint8)
        lib.oracle_attention_masked(_ptr(out), _ptr(q), _ptr(k), _ptr(v), seq, heads, 128, scale, _ptr(m), block, r0, r1)
    return out


def attention_f64(q, k, v, seq, heads, scale, rows=None):
    lib = load()
    r0, r1 = rows if rows is not None else (0, seq)
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros((r1 - r0, heads, 128), dtype=np.float64)
    lib.oracle_attention_f64(_ptr(out), _ptr(q), _ptr(k), _ptr(v), seq, heads, 128, float(scale), r0, r1)
    return out


def sage_pack(q, k, v, seq, heads):
    lib = load()
    padded = (seq + 63) // 64 * 64
    blocks = padded // 64
    q, k, v = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k, v))
    q8 = np.zeros(heads * padded * 128, np.int8)
    k8 = np.zeros_like(q8)
    v8 = np.zeros(heads * padded * 128, np.uint8)
    qs = np.zeros(heads * blocks, np.float32)
    ks = np.zeros_like(qs)
    vs = np.zeros(heads * 128, np.float32)
    km = np.zeros(heads * 128, np.uint16)
    lib.oracle_sage_pack(_ptr(q), _ptr(k), _ptr(v), seq, heads, _ptr(q8), _ptr(k8), _ptr(v8),
                         _ptr(qs), _ptr(ks), _ptr(vs), _ptr(km))
    return dict(q8=q8, k8=k8, v8=v8, q_scale=qs, k_scale=ks, v_scale=vs, k_mean=km)


def k_mean_f64(k, seq, heads):
    lib = load()
    k = np.ascontiguousarray(k, dtype=np.uint16)
    out = np.zeros(heads * 128, np.float64)
    lib.oracle_k_mean_f64(_ptr(k), seq, heads, _ptr(out))
    return out


def sage_attention(pack, seq, heads, scale, rows=None, mask=None, block=128):
    lib = load()
    r0, r1 = rows if rows is not None else (0, seq)
    out = np.zeros((r1 - r0, heads, 128), np.float64)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    lib.oracle_sage_attention(_ptr(out), _ptr(pack["q8"]), _ptr(pack["k8"]), _ptr(pack["v8"]),
                              _ptr(pack["q_scale"]), _ptr(pack["k_scale"]), _ptr(pack["v_scale"]),
                              seq, heads, scale, _ptr(m), block, r0, r1)
    return out


def e4m3_encode(x):
    lib = load()
    return np.array([lib.oracle_f32_to_e4m3(float(t)) for t in np.asarray(x, np.float32).reshape(-1)], np.uint8)


def e4m3_decode(codes):
    lib = load()
    return np.array([lib.oracle_e4m3_to_f32(int(c)) for c in np.asarray(codes, np.uint8).reshape(-1)], np.float32)


def sage_v_position(j):
    return load().oracle_sage_v_position(j)


def threads():
    return load().oracle_threads()


def xorshift_bf16(count, seed_state):
    """Reference attention test inputs (tests/cuda_attention.c:14-18). seed_state
    is a one-element uint32 array advanced in place."""
    out = np.empty(count, np.uint16)
    load().oracle_xorshift_bf16(_ptr(out), count, seed_state.ctypes.data)
    return out


def xorshift_native_bf16(count, state):
    """Reference Sage/native test inputs (tests/attention_native.c:20,56)."""
    out = np.empty(count, np.uint16)
    load().oracle_xorshift_native_bf16(_ptr(out), count, state.ctypes.data)
    return out


def block_mask(seq, video_rows, block, density, seed):
    """Synthetic block mask, restated in numpy from its
    definition: diagonal, audio<->audio block pairs, and a seeded Bernoulli(density)
    draw u = (splitmix64((seed << 40) + qb*B + kb) >> 11) * 2^-53 < density."""
    blocks = (seq + block - 1) // block
    qb, kb = np.meshgrid(np.arange(blocks, dtype=np.uint64), np.arange(blocks, dtype=np.uint64), indexing="ij")
    z = (np.uint64(seed) << np.uint64(40)) + qb * np.uint64(blocks) + kb
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = (z >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    last = np.arange(blocks) * block + block - 1
    audio = (last >= video_rows) & (video_rows < seq)
    keep = (qb == kb) | (audio[:, None] & audio[None, :]) | (u < density)
    return keep.astype(np.uint8)
