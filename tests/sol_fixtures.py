"""SOL fixtures and the reference's independent NumPy oracle formulas
(tests/cuda_sol_oracle.py:11-56): block metadata with protected rows, float32
summaries, float64 routes and the float64 exact + centroid softmax. They check
the C restatement in oracle/sol.c and the HIP SOL path."""
import numpy as np

from h3cli_amd import synth


def metadata(seq, qb, protected=False, all_protected=False):
    """int32 [blocks, 4] (protect, first_frame, last_frame, rows) for q blocks of
    qb rows and 64-row key blocks (cuda_sol_oracle.py:15-22): protected rows are
    the first 17, the last 19 and the block holding seq // 2; frames are
    row // 128 when protected, else -1."""
    result = []
    for block in (qb, 64):
        blocks = []
        for start in range(0, seq, block):
            end = min(seq, start + block)
            protect = all_protected or (protected and (start < 17 or end > seq - 19 or start <= seq // 2 < end))
            blocks.append([int(protect), start // 128 if protected else -1, (end - 1) // 128 if protected else -1,
                           end - start])
        result.append(np.array(blocks, dtype=np.int32))
    return result


def inputs(seq, heads, seed=1701, pattern="random"):
    """BF16 bits Q, K, V [seq, heads, 128] (cuda_sol_oracle.py:66-74 patterns)."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, .5, (3, seq, heads, 128)).astype(np.float32)
    if pattern == "zero":
        x[:] = 0
    elif pattern == "constant":
        x[1] = .2
        x[2] = .7
    elif pattern == "extreme":
        x[:2] *= 40
    elif pattern == "spike":
        x[1, seq // 2] *= 32
    elif pattern == "nan":
        x[0, -1, -1, 0] = np.nan
    return [synth.f32_to_bf16(a) for a in x]


def summaries(x, b):
    """float32 mean per block (numpy's summation), BF16-rounded."""
    xf = synth.bf16_to_f32(x)
    return synth.bf16_to_f32(synth.f32_to_bf16(
        np.array([xf[i:i + b].mean(axis=0, dtype=np.float32) for i in range(0, len(xf), b)])))


def routes64(qc, kc, meta, scale, minimum, tau, radius, exact=False):
    """float64 routes of one head (cuda_sol_oracle.py:27-40); also returns the
    float64 dots and thresholds."""
    qm, km = meta
    count = len(km)
    mu = kc.mean(axis=0, dtype=np.float64)
    var = np.maximum((kc.astype(np.float64) ** 2).mean(axis=0) - mu * mu, 0)
    a = scale * np.log2(np.e)
    threshold = qc @ mu * a + tau * np.sqrt(((qc.astype(np.float64) ** 2) @ var) * a * a + 1e-6)
    dots = qc.astype(np.float64) @ kc.astype(np.float64).T * a
    route = dots > threshold[:, None]
    route |= ~np.isfinite(dots) | ~np.isfinite(threshold[:, None])
    route |= bool(exact)
    route |= (qm[:, 0] != 0)[:, None] | (km[:, 0] != 0)[None, :]
    local = ((qm[:, 1, None] >= 0) & (km[None, :, 1] >= 0) & (qm[:, 1, None] <= km[None, :, 2] + radius) &
             (km[None, :, 1] <= qm[:, 2, None] + radius))
    floor = int(np.ceil(float(np.float32(minimum)) * count))
    idx = np.arange(count, dtype=np.int64)
    route |= local | (((idx + 1) * floor // count) != (idx * floor // count))[None, :] | (km[:, 3] < 64)[None, :]
    return route, dots, threshold


def attention64(q, k, v, kc, vc, route, qb, scale, rows, head):
    """float64 softmax over exact keys and biased centroid entries for `rows`
    of one head (cuda_sol_oracle.py:43-56). q, k, v: float32 [seq, heads, 128];
    kc, vc: float32 [kblocks, 128] of this head; route [qblocks, kblocks]."""
    seq = q.shape[0]
    out = np.empty((len(rows), 128))
    for i, r in enumerate(rows):
        rb = route[r // qb]
        exact_rows = np.repeat(rb.astype(bool), 64)[:seq]
        keys = np.concatenate((k[exact_rows, head], kc[~rb.astype(bool)])).astype(np.float64)
        values = np.concatenate((v[exact_rows, head], vc[~rb.astype(bool)])).astype(np.float64)
        s = keys @ q[r, head].astype(np.float64) * scale
        s[int(exact_rows.sum()):] += np.log(64.)
        s -= s.max()
        p = np.exp(s)
        out[i] = p @ values / p.sum()
    return out
