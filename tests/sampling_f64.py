"""Float64 restatement of the stochastic branch of sample_impl (tl_cpu tensor.rs:1641-1679),
shared by the oracle's and the GPU's sampling tests.

The reference adds probabilities in f32 in sorted order, so its cutoff and its choice can
move where top_p or r = u * cutoff lies within that rounding of a running sum.  sample_f64
returns the choice with exact (float64) running sums, the distance of top_p and r from the
nearest running sum (margin), and the largest gap between f32 sequential running sums and
the float64 ones (drift): a choice is decided the same way by every correct summation when
margin > 4e-6 + 4 * drift (4e-6 covers the f32 rounding of the probabilities themselves).
bracketed() checks any choice against the definition instead: its place in the float64
order has running sums that bracket r within a tolerance, for a cutoff anywhere top_p could
fall within that tolerance -- for flat distributions over many elements, whose running sums
lie closer together than any summation's rounding.
"""
import numpy as np


def sample_f64(x, temp, top_p, u):
    p = (np.asarray(x, np.float32).ravel() / np.float32(temp)).astype(np.float64)
    e = np.exp(p - p.max())
    pr = e / e.sum()
    order = np.argsort(-pr, kind="stable")  # descending, equal probs in index order
    cs = np.cumsum(pr[order])
    over = np.nonzero(cs > top_p)[0]
    c = int(over[0]) if len(over) else len(cs) - 1
    r = float(np.float32(u)) * cs[c]
    hit = np.nonzero(cs[:c + 1] >= r)[0]
    sel = int(order[hit[0]]) if len(hit) else int(order[0])
    m_cut = np.abs(cs - top_p).min() if np.isfinite(top_p) else np.inf
    margin = min(m_cut, np.abs(cs[:c + 1] - r).min())
    cs32 = np.cumsum(pr[order].astype(np.float32), dtype=np.float32)  # sequential f32 sums
    drift = float(np.abs(cs32.astype(np.float64) - cs).max())
    return sel, float(margin), drift


def decided(margin, drift):
    return margin > 4e-6 + 4 * drift


def bracketed(x, temp, top_p, u, got, tol=4e-6):
    p = (np.asarray(x, np.float32).ravel() / np.float32(temp)).astype(np.float64)
    e = np.exp(p - p.max())
    pr = e / e.sum()
    order = np.argsort(-pr, kind="stable")
    cs = np.cumsum(pr[order])
    pos = int(np.nonzero(order == got)[0][0])
    if not np.isfinite(top_p):
        cuts = [len(cs) - 1]
    else:  # every place the cutoff could take within tol of top_p
        lo = np.nonzero(cs > top_p - tol)[0]
        hi = np.nonzero(cs > top_p + tol)[0]
        c_lo = int(lo[0]) if len(lo) else len(cs) - 1
        c_hi = int(hi[0]) if len(hi) else len(cs) - 1
        cuts = range(c_lo, c_hi + 1)
    before = cs[pos - 1] if pos else 0.0
    for c in cuts:
        r = float(np.float32(u)) * cs[c]
        if pos <= c and before < r + tol and cs[pos] >= r - tol:
            return True
        if pos == 0 and r > cs[c] - tol:  # no running sum reaches r: order[0]
            return True
    return False


def splitmix64_uniforms(seed, count):
    """The draws of tl_hip_tensor_sample after tl_hip_sample_seed(seed): splitmix64, top 53
    bits times 2^-53 (the published splitmix64 constants)."""
    mask = (1 << 64) - 1
    s, out = seed & mask, []
    for _ in range(count):
        s = (s + 0x9E3779B97F4A7C15) & mask
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        z ^= z >> 31
        out.append((z >> 11) * 2.0 ** -53)
    return out
