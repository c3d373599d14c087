"""Input generators and comparisons shared by the tests."""
import numpy as np


def lcg(seed: int):
    """The reference tests' generator (transformer.rs:1116-1124): an LCG step, then
    (seed >> 40) / 2^24 - 0.5, uniform in [-0.5, 0.5)."""
    state = [seed & 0xFFFFFFFFFFFFFFFF]

    def rand(n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        s = state[0]
        for i in range(n):
            s = (s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
            out[i] = np.float32((s >> 40) / float(1 << 24) - 0.5)
        state[0] = s
        return out

    return rand


def bf16_round(a) -> np.ndarray:
    """Round-to-nearest-even to bf16 on the f32 bits (finite inputs)."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(a.shape)


def normal(rng: np.random.Generator, shape, act: str) -> np.ndarray:
    x = rng.standard_normal(shape).astype(np.float32)
    return bf16_round(x) if act == "bf16" else x


def rel_err(got, want) -> float:
    """max |got - want| over max |want|, per (row, head) vector; the worst of them."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    num = np.abs(got - want).max(axis=-1)
    den = np.maximum(np.abs(want).max(axis=-1), 1e-30)
    return float((num / den).max())


def rope_f64(x, pos, theta=10000.0):
    """x [n][H][64] rotated at positions pos [n] in f64, pairs (2i, 2i + 1) by pos / theta^(i / 32)
    (rope.rs:44-58, 74-95, with exact angles)."""
    x = np.asarray(x, np.float64)
    inv = theta ** (-np.arange(32, dtype=np.float64) / 32.0)
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s_ = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s_
    out[..., 1::2] = x0 * s_ + x1 * c
    return out


def exact_attend(q, keys, vals, scale=0.125):
    """One query row [H][64] over the rows of a sequence (keys and values [n][H][64], before RoPE,
    at positions 0 .. n - 1; the query at n - 1), in f64: the mathematics every mode approximates."""
    n = keys.shape[0]
    qr = rope_f64(q[None], [n - 1])[0]
    kr = rope_f64(keys, np.arange(n))
    sc = np.einsum("hd,nhd->hn", qr, kr) * scale
    w = np.exp(sc - sc.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    return np.einsum("hn,nhd->hd", w, np.asarray(vals, np.float64))
