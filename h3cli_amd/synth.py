"""Seeded synthetic inputs for the BASELINE configurations (host side, numpy).

Generator (documented so any implementation can reproduce it):
    splitmix64(x): z = x + 0x9E3779B97F4A7C15;
                   z = (z ^ z>>30) * 0xBF58476D1CE4E5B9;
                   z = (z ^ z>>27) * 0x94D049BB133111EB;  return z ^ z>>31   (mod 2^64)
    normal(seed, 2j), normal(seed, 2j+1) — Box-Muller on
        a = splitmix64((seed << 40) + 2j), b = splitmix64((seed << 40) + 2j + 1),
        u1 = ((a >> 11) + 1) * 2^-53, u2 = (b >> 11) * 2^-53,
        r = sqrt(-2 ln u1): (r cos 2 pi u2, r sin 2 pi u2), in float64.
The device fill kernel (h3_hip_fill_normal_bf16) uses the same formula.
"""
import numpy as np

_M1 = np.uint64(0x9E3779B97F4A7C15)
_M2 = np.uint64(0xBF58476D1CE4E5B9)
_M3 = np.uint64(0x94D049BB133111EB)


def splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x.astype(np.uint64) + _M1
        z = (z ^ (z >> np.uint64(30))) * _M2
        z = (z ^ (z >> np.uint64(27))) * _M3
        return z ^ (z >> np.uint64(31))


def normal(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """float64 N(0,1) values [offset, offset+count) of stream `seed`."""
    first_pair = offset // 2
    pairs = (offset + count + 1) // 2 - first_pair
    j = np.arange(first_pair, first_pair + pairs, dtype=np.uint64)
    base = np.uint64(seed) << np.uint64(40)
    with np.errstate(over="ignore"):
        a = splitmix64(base + np.uint64(2) * j)
        b = splitmix64(base + np.uint64(2) * j + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, dtype=np.float64)
    out[0::2] = r * np.cos(2 * np.pi * u2)
    out[1::2] = r * np.sin(2 * np.pi * u2)
    start = offset - 2 * first_pair
    return out[start:start + count]


def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16); NaN stays NaN."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r.reshape(np.shape(x))


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def normal_bf16(seed: int, count: int, scale: float = 1.0) -> np.ndarray:
    return f32_to_bf16((normal(seed, count) * scale).astype(np.float32))


def rope_tables(frames: int, height: int, width: int, split=(44, 42, 42), theta: float = 10000.0):
    """3D RoPE cos/sin [frames*height*width, 64] (float32) for the rotate-half
    convention of the reference's qkv_rope (pair d <-> d + 64). Pair j belongs to
    axis a with i = j - start_a; angle = pos_a * theta^(-2 i / dim_a). Token order
    is frame-major, then row, then column."""
    pairs = [d // 2 for d in split]
    tt, hh, ww = np.meshgrid(np.arange(frames), np.arange(height), np.arange(width), indexing="ij")
    pos = [tt.reshape(-1), hh.reshape(-1), ww.reshape(-1)]
    cols = []
    for a, (dim, count) in enumerate(zip(split, pairs)):
        inv = theta ** (-2.0 * np.arange(count, dtype=np.float64) / dim)
        cols.append(pos[a][:, None].astype(np.float64) * inv[None, :])
    ang = np.concatenate(cols, axis=1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE on [S, H, 128] float32 with cos/sin [S, 64] (rounded to
    bf16 first, as the reference's tables are): y[d] = x[d] c - x[d+64] s,
    y[d+64] = x[d+64] c + x[d] s."""
    c = bf16_to_f32(f32_to_bf16(cos))[:, None, :]
    s = bf16_to_f32(f32_to_bf16(sin))[:, None, :]
    lo, hi = x[..., :64], x[..., 64:]
    return np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=-1).astype(np.float32)


def attention_inputs(seq: int, heads: int, seed: int = 0, scale: float = 0.5, rope_shape=None):
    """bf16 Q, K, V [seq, heads, 128] from N(0,1)*scale; with rope_shape (t,h,w)
    the 3D RoPE is applied to Q and K."""
    n = seq * heads * 128
    out = []
    for i in range(3):
        x = (normal(seed * 16 + i, n) * scale).astype(np.float32).reshape(seq, heads, 128)
        x = bf16_to_f32(f32_to_bf16(x))
        if rope_shape is not None and i < 2:
            cos, sin = rope_tables(*rope_shape)
            x = apply_rope(x, cos[:seq], sin[:seq])
        out.append(f32_to_bf16(x))
    return out
