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
        lib.oracle_q8_pack.argtypes = [_p, _p, _p, _u, _u, _u]
        lib.oracle_linear_q8.argtypes = [_p, _p, _p, _p, _p, _p, _u, _u, _u, _u, C.c_int, _u, _u]
        lib.oracle_linear_bf16.argtypes = [_p, _p, _p, _p, _p, _u, _u, _u, C.c_int, _u, _u]
        lib.oracle_adaln.argtypes = [_p, _p, _p, _p, _p, _u, _u, _u, _u, _u, _f]
        lib.oracle_gate.argtypes = [_p, _p, _p, _p, _p, _u, _u, _u, _u]
        lib.oracle_qkv_rope.argtypes = [_p, _p, _p, _p, _p, _p, _p, _p, _u, _u, _u, _u, _f, C.c_int]
        lib.oracle_gelu.argtypes = [_p, _p, C.c_size_t, C.c_int]
        lib.oracle_gelu_tanh.argtypes = [_f]
        lib.oracle_gelu_tanh.restype = _f
        lib.oracle_swiglu.argtypes = [_p, _p, _u, _u]
        lib.oracle_euler.argtypes = [_p, _p, _p, C.c_size_t, _f, _f]
        lib.oracle_rms_norm.argtypes = [_p, _p, _p, _u, _u, _f]
        lib.oracle_sb_pool.argtypes = [_p, _p, _u, _u, _f]
        lib.oracle_sol_summary.argtypes = [_p, _p, _u, _u, _u]
        lib.oracle_sol_moments.argtypes = [_p, _p, _u, _u]
        lib.oracle_sol_route.argtypes = [_p, _p, _p, _p, _p, _p, _p, _u, _u, _u, _u, _u, _f, _f, C.c_int]
        lib.oracle_sol_attention.argtypes = [_p, _p, _p, _p, _p, _p, _p, _u, _u, _u, _f, _u, _u]
        lib.oracle_sb_score.argtypes = [_p, _p, _p, _u, _u]
        lib.oracle_sb_select.argtypes = [_p, _p, _u, _u, _u, _p, _p]
        lib.oracle_attention_routed.argtypes = [_p, _p, _p, _p, _u, _u, _f, _p, _u, _u]
        lib.oracle_head_rms_norm.argtypes = [_p, _p, _u, _u, _u, _f]
        lib.oracle_patch_linear.argtypes = [_p, _p, _p, _p, _p, _u, _u, _u, _u]
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


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def q8_pack(w, rows, cols, group=64):
    """Reference q8 packing (src/weights/q8.c:26-56) with a group parameter."""
    w = _u16(w)
    groups = (cols + group - 1) // group
    codes = np.zeros(rows * cols, np.int8)
    scales = np.zeros(rows * groups, np.float32)
    ok = load().oracle_q8_pack(_ptr(w), _ptr(codes), _ptr(scales), rows, cols, group)
    return (codes, scales) if ok else None


def linear_q8(x, codes, scales, rows, k, n, group, bias=None, gelu=False, rows_range=None):
    r0, r1 = rows_range if rows_range else (0, rows)
    y = np.zeros((r1 - r0) * n, np.uint16)
    y64 = np.zeros((r1 - r0) * n, np.float64)
    b = None if bias is None else _u16(bias)
    load().oracle_linear_q8(_ptr(y), _ptr(y64), _ptr(_u16(x)), _ptr(np.ascontiguousarray(codes, np.int8)),
                            _ptr(np.ascontiguousarray(scales, np.float32)), _ptr(b), rows, k, n, group,
                            int(gelu), r0, r1)
    return y, y64


def linear_bf16(x, w, rows, k, n, bias=None, gelu=False, rows_range=None):
    r0, r1 = rows_range if rows_range else (0, rows)
    y = np.zeros((r1 - r0) * n, np.uint16)
    y64 = np.zeros((r1 - r0) * n, np.float64)
    b = None if bias is None else _u16(bias)
    load().oracle_linear_bf16(_ptr(y), _ptr(y64), _ptr(_u16(x)), _ptr(_u16(w)), _ptr(b), rows, k, n, int(gelu), r0, r1)
    return y, y64


def adaln(x, w, mod, row_map, rows, width, slots, shift, scale, eps):
    y = np.zeros(rows * width, np.uint16)
    load().oracle_adaln(_ptr(y), _ptr(_u16(x)), _ptr(_u16(w)), _ptr(_u16(mod)),
                        _ptr(np.ascontiguousarray(row_map, np.uint32)), rows, width, slots, shift, scale, eps)
    return y


def gate(res, branch, mod, row_map, rows, width, slots, gate_slot):
    y = np.zeros(rows * width, np.uint16)
    load().oracle_gate(_ptr(y), _ptr(_u16(res)), _ptr(_u16(branch)), _ptr(_u16(mod)),
                       _ptr(np.ascontiguousarray(row_map, np.uint32)), rows, width, slots, gate_slot)
    return y


def qkv_rope(qkv, qw, kw, cos_t, sin_t, seq, heads, dim, half, eps, grouped):
    n = seq * heads * dim
    q, k, v = (np.zeros(n, np.uint16) for _ in range(3))
    load().oracle_qkv_rope(_ptr(q), _ptr(k), _ptr(v), _ptr(_u16(qkv)), _ptr(None if qw is None else _u16(qw)),
                           _ptr(None if kw is None else _u16(kw)), _ptr(_u16(cos_t)), _ptr(_u16(sin_t)),
                           seq, heads, dim, half, eps, int(grouped))
    return q, k, v


def gelu(x, approximate=True):
    x = _u16(x)
    y = np.zeros(x.size, np.uint16)
    load().oracle_gelu(_ptr(y), _ptr(x), x.size, int(approximate))
    return y


def swiglu(fused, rows, width):
    y = np.zeros(rows * width, np.uint16)
    load().oracle_swiglu(_ptr(y), _ptr(_u16(fused)), rows, width)
    return y


def euler(sample, last, previous, delta, ratio):
    s = np.array(sample, np.float32, copy=True)
    load().oracle_euler(_ptr(s), _ptr(_u16(last)), _ptr(_u16(previous)), s.size, delta, ratio)
    return s


def rms_norm(x, w, rows, width, eps):
    y = np.zeros(rows * width, np.uint16)
    load().oracle_rms_norm(_ptr(y), _ptr(_u16(x)), _ptr(_u16(w)), rows, width, eps)
    return y


def head_rms_norm(t, w, seq, heads, dim, eps):
    y = np.array(_u16(t), copy=True)
    load().oracle_head_rms_norm(_ptr(y), _ptr(_u16(w)), seq, heads, dim, eps)
    return y


def patch_linear(x, w, bias, m, k, n, row_map=None, out_rows=None):
    out_rows = m if out_rows is None else out_rows
    y = np.zeros(out_rows * n, np.uint16)
    xf = np.ascontiguousarray(x, np.float32)
    wf = np.ascontiguousarray(w, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    mp = None if row_map is None else np.ascontiguousarray(row_map, np.uint32)
    load().oracle_patch_linear(_ptr(y), _ptr(xf), _ptr(wf), _ptr(b), _ptr(mp), out_rows, m, k, n)
    return y


def sb_pool(x, seq, heads, scale):
    cells = (seq + 63) // 64 * 4
    out = np.zeros(heads * cells * 128, np.uint16)
    load().oracle_sb_pool(_ptr(out), _ptr(_u16(x)), seq, heads, scale)
    return out


def sb_score(qp, kp, seq, heads):
    blocks = (seq + 63) // 64
    out = np.zeros(heads * blocks * blocks, np.float32)
    load().oracle_sb_score(_ptr(out), _ptr(_u16(qp)), _ptr(_u16(kp)), seq, heads)
    return out


def sb_select(scores, heads, blocks, keep, q_protect=None, k_protect=None):
    routes = np.zeros(heads * blocks * blocks, np.uint8)
    qp = None if q_protect is None else np.ascontiguousarray(q_protect, np.uint8)
    kp = None if k_protect is None else np.ascontiguousarray(k_protect, np.uint8)
    load().oracle_sb_select(_ptr(routes), _ptr(np.ascontiguousarray(scores, np.float32)), heads, blocks, keep,
                            _ptr(qp), _ptr(kp))
    return routes


def attention_routed(q, k, v, seq, heads, scale, routes, rows=None):
    r0, r1 = rows or (0, seq)
    out = np.zeros((r1 - r0) * heads * 128, np.float32)
    load().oracle_attention_routed(_ptr(out), _ptr(_f32(q)), _ptr(_f32(k)), _ptr(_f32(v)), seq, heads, scale,
                                   _ptr(np.ascontiguousarray(routes, np.uint8)), r0, r1)
    return out


def sol_summary(x, seq, heads, block):
    blocks = (seq + block - 1) // block
    out = np.zeros(heads * blocks * 128, np.uint16)
    load().oracle_sol_summary(_ptr(out), _ptr(_u16(x)), seq, heads, block)
    return out


def sol_moments(kc, heads, blocks):
    out = np.zeros(heads * 256, np.float32)
    load().oracle_sol_moments(_ptr(out), _ptr(_u16(kc)), heads, blocks)
    return out


def sol_route(qc, kc, moments, qmeta, kmeta, heads, radius, minimum, scale, tau, force_exact=False):
    """qmeta/kmeta: int32 [blocks, 4] (protect, first_frame, last_frame, rows).
    Returns (routes u8 [heads, qblocks, kblocks], counts[7])."""
    qm = np.ascontiguousarray(qmeta, np.int32)
    km = np.ascontiguousarray(kmeta, np.int32)
    qb, kb = len(qm), len(km)
    routes = np.zeros(heads * qb * kb, np.uint8)
    counts = np.zeros(7, np.uint64)
    load().oracle_sol_route(_ptr(routes), _ptr(counts), _ptr(_u16(qc)), _ptr(_u16(kc)),
                            _ptr(np.ascontiguousarray(moments, np.float32)), _ptr(qm), _ptr(km), heads, qb, kb,
                            radius, minimum, scale, tau, int(force_exact))
    return routes.reshape(heads, qb, kb), counts


def sol_attention(q, k, v, kc, vc, routes, seq, heads, qblock, scale, rows=None):
    r0, r1 = rows or (0, seq)
    out = np.zeros((r1 - r0) * heads * 128, np.float32)
    load().oracle_sol_attention(_ptr(out), _ptr(_u16(q)), _ptr(_u16(k)), _ptr(_u16(v)), _ptr(_u16(kc)),
                                _ptr(_u16(vc)), _ptr(np.ascontiguousarray(routes, np.uint8)), seq, heads, qblock,
                                scale, r0, r1)
    return out


def fp8_pack(x, count=None, padded=None):
    """Tensorwide E4M3 packing (cuda_quant.cuh:26-49). Returns (codes u8
    [padded], scale f32, nonfinite)."""
    x = _u16(x).reshape(-1)
    count = x.size if count is None else count
    padded = count if padded is None else padded
    codes = np.zeros(padded, np.uint8)
    scale = np.zeros(1, np.float32)
    lib = load()
    lib.oracle_fp8_pack.restype = C.c_int
    lib.oracle_fp8_pack.argtypes = [_p, _p, _p, C.c_size_t, C.c_size_t]
    bad = lib.oracle_fp8_pack(_ptr(codes), _ptr(scale), _ptr(x), count, padded)
    return codes, np.float32(scale[0]), bool(bad)


def fp8_gemm(x8, sx, w8, sw, m, n, k):
    """y [m, n] BF16 bits = bf16(sx * sw * sum x8 . w8^T) (cuda_quant.cuh:362-394)."""
    y = np.zeros(m * n, np.uint16)
    lib = load()
    lib.oracle_fp8_gemm.argtypes = [_p, _p, C.c_float, _p, C.c_float, _u, _u, _u]
    lib.oracle_fp8_gemm(_ptr(y), _ptr(np.ascontiguousarray(x8, np.uint8)), float(sx),
                        _ptr(np.ascontiguousarray(w8, np.uint8)), float(sw), m, n, k)
    return y.reshape(m, n)


def nvfp4_scale_bytes(rows, k):
    """Bytes of the VEC16 tiled scale plane (cuda_quant.cuh:14-16)."""
    return ((rows + 127) // 128 * 128) * ((k // 16 + 3) // 4 * 4)


def nvfp4_pack(x, rows, k, padded=None, weight_global=0.0):
    """NVFP4 packing (cuda_quant.cuh:50-72). Returns (codes u8 [padded*k/2],
    scales u8 tiled plane, global f32[4], nonfinite)."""
    x = _u16(x).reshape(-1)
    padded = rows if padded is None else padded
    codes = np.zeros(padded * k // 2, np.uint8)
    scales = np.zeros(nvfp4_scale_bytes(padded, k), np.uint8)
    glob = np.zeros(4, np.float32)
    lib = load()
    lib.oracle_nvfp4_pack.restype = C.c_int
    lib.oracle_nvfp4_pack.argtypes = [_p, _p, _p, _p, _u, _u, _u, C.c_float]
    bad = lib.oracle_nvfp4_pack(_ptr(codes), _ptr(scales), _ptr(glob), _ptr(x), rows, padded, k, float(weight_global))
    return codes, scales, glob, bool(bad)


def nvfp4_gemm(x4, xs, w4, ws, alpha, m, n, k):
    y = np.zeros(m * n, np.uint16)
    lib = load()
    lib.oracle_nvfp4_gemm.argtypes = [_p, _p, _p, _p, _p, C.c_float, _u, _u, _u]
    lib.oracle_nvfp4_gemm(_ptr(y), _ptr(np.ascontiguousarray(x4, np.uint8)), _ptr(np.ascontiguousarray(xs, np.uint8)),
                          _ptr(np.ascontiguousarray(w4, np.uint8)), _ptr(np.ascontiguousarray(ws, np.uint8)),
                          float(alpha), m, n, k)
    return y.reshape(m, n)


def e2m1_decode(codes):
    lib = load()
    lib.oracle_e2m1_to_f32.restype = C.c_float
    lib.oracle_e2m1_to_f32.argtypes = [C.c_uint8]
    return np.array([lib.oracle_e2m1_to_f32(int(c)) for c in np.asarray(codes).reshape(-1)], np.float32)


def nvfp4_scale_index(row, block, k):
    lib = load()
    lib.oracle_nvfp4_scale_index.restype = C.c_size_t
    lib.oracle_nvfp4_scale_index.argtypes = [_u, _u, _u]
    return lib.oracle_nvfp4_scale_index(row, block, k)
