"""Seeded synthetic inputs for the tests (numpy on the host).

Rows are drawn from N(0, 1) in fp32, scaled to unit RMS per row (x / sqrt(mean(x^2)
+ 1e-6), mimicking QK-norm / V-norm) and rounded to bf16 (round-to-nearest-even).
"""
import numpy as np

from oracle import oracle as orc

EPS = 1e-6
_CHUNK_ROWS = 1 << 16


def rms_rows(rng: np.random.Generator, shape) -> np.ndarray:
    shape = tuple(shape)
    D = shape[-1]
    n_rows = int(np.prod(shape[:-1])) if len(shape) > 1 else 1
    out = np.empty((n_rows, D), dtype=np.uint16)
    for r0 in range(0, n_rows, _CHUNK_ROWS):
        r1 = min(n_rows, r0 + _CHUNK_ROWS)
        x = rng.standard_normal(size=(r1 - r0, D), dtype=np.float32)
        r = np.sqrt(np.mean(x * x, axis=-1, keepdims=True, dtype=np.float64) + EPS)
        out[r0:r1] = orc.to_bf16((x / r).astype(np.float32))
    return out.reshape(shape)


def pooled_rows(rng: np.random.Generator, n_rows: int, D: int, pool: int) -> np.ndarray:
    """n_rows unit-RMS bf16 rows, each a random pick from `pool` distinct rows: multi-GB
    caches in seconds.  With a pool of 65536, a row read from the wrong place differs
    from the right one with probability 1 - 2^-16."""
    table = rms_rows(rng, (pool, D))
    return table[rng.integers(0, pool, size=n_rows)]


def make_step_inputs(step: orc.Step, seed: int, pos, shared_kv: bool = False, row_base=None,
                     pool: int = 0):
    """Random q, flat caches and new rows for one decode step.

    Every cache element is filled (rows that are not visible hold data too, so a kernel
    that reads them by mistake changes the result).  pool > 0 draws the cache rows from
    `pool` distinct rows (pooled_rows)."""
    rng = np.random.default_rng(seed)
    d = step.desc()
    q = rms_rows(rng, (step.B, step.Hq, step.D))
    n_elems = int(d.seq_stride) * step.B

    def cache():
        if pool:
            return pooled_rows(rng, n_elems // step.D, step.D, pool).reshape(-1)
        return rms_rows(rng, (n_elems // step.D, step.D)).reshape(-1)

    kc = cache()
    vc = kc if shared_kv else cache()
    kn = rms_rows(rng, (step.B, step.Hkv, step.D))
    vn = kn if shared_kv else rms_rows(rng, (step.B, step.Hkv, step.D))
    return q, kc, vc, kn, vn


def plant_peaked_keys(step: orc.Step, q, kc, pos, n_peaks: int, bump: float, seed: int,
                      row_base=None):
    """Add bump * q_hat to n_peaks visible keys per (sequence, kv head), where q_hat is
    the unit direction of the group's first query head; with scale * |q| = 1 (unit-RMS
    q, scale 1/sqrt(D)) that head's logit rises by exactly `bump` before bf16 rounding.
    Returns the planted absolute positions per sequence."""
    rng = np.random.default_rng(seed)
    d = step.desc()
    G = step.Hq // step.Hkv
    planted = []
    for b in range(step.B):
        rows = orc.visible(step, pos[b], 0 if row_base is None else row_base[b])
        pick = rng.choice(len(rows), size=min(n_peaks, len(rows)), replace=False)
        planted.append(sorted(int(x) for x in pick))
        for h in range(step.Hkv):
            qh = orc.from_bf16(q[b, h * G]).astype(np.float64)
            qhat = qh / np.linalg.norm(qh)
            alpha = bump / (step.scale * np.linalg.norm(qh))
            base = b * d.seq_stride + h * d.head_stride
            for t in pick:
                o = base + int(rows[t]) * step.D
                k = orc.from_bf16(kc[o:o + step.D]).astype(np.float64) + alpha * qhat
                kc[o:o + step.D] = orc.to_bf16(k.astype(np.float32))
    return planted
