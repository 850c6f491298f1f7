"""Oracle for the fused sampler and its uniforms (test infrastructure only).

``sample`` restates the sampler contract step by step in float32 so the
token ids of the HIP kernel can be checked bit for bit.  The contract follows
the reference's fused code-predictor sampler (executor/sampling.py:242-302)
with an explicit uniform in place of ``tl.rand(seed, offset)``, plus the
penalty / greedy / masking rules of model/sampling.py:55-65,183-187 and
executor/talker.py:173-183,240-243:

    x      = logits (fp32); masked ids -> -inf; seen ids: x>0 ? x/r : x*r
    T == 0 -> argmax x (lowest id on ties)
    s      = x / T; ranks ordered by (s desc, id asc) on the sortable bit key
    k_eff  = k > 0 ? min(k, V) : V;  w_r = nq_exp(s_r - s_0)
    cum    = segmented 64-lane scan (see ``wave_scan``)
    keep   = longest prefix with (cum_r - w_r) < min(p,1) * cum_{k-1}
    token  = first kept rank with cum_r >= u * cum_{kept-1}, else the last kept

``nq_exp`` is Cody-Waite range reduction with Cephes' two-part ln 2 and a
degree-7 Taylor polynomial, every step an IEEE float32 operation.

``philox4x32`` is Philox-4x32-10 (Salmon et al., SC'11) and
``uniform_from_counter`` the (seed, offset) -> u map of the HIP library.

Pinned by tests/test_oracle_sampler.py: Random123's published Philox
known-answer vectors, nq_exp against float64 exp (<= 2 ulp), the scan against
exact integer sums, special cases (T = 0 argmax, k = 1, u = 0, tiny p,
one-hot logits) and a float64 inverse-CDF restatement of the reference's
fused sampler that must agree except where u lies within 1e-5 of a
cumulative boundary.
"""

from __future__ import annotations

import numpy as np

F = np.float32
_LOG2E = np.uint32(0x3FB8AA3B).view(np.float32)
_LN2_HI = np.uint32(0x3F318000).view(np.float32)
_LN2_LO = np.uint32(0xB95E8083).view(np.float32)
_EXP_LOW = np.uint32(0xC2AE0000).view(np.float32)
_TAYLOR = [F(1.0) / F(5040.0), F(1.0) / F(720.0), F(1.0) / F(120.0), F(1.0) / F(24.0),
           F(1.0) / F(6.0), F(0.5), F(1.0), F(1.0)]


def nq_exp(x: np.ndarray) -> np.ndarray:
    """The sampler's exp, float32 in and out, bit-identical to the kernel."""

    x = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        low = ~(x > _EXP_LOW)
        xs = np.where(low, F(0.0), x).astype(np.float32)
        t = (xs * _LOG2E).astype(np.float32)
        n = np.floor((t + F(0.5)).astype(np.float32)).astype(np.float32)
        r = (xs - (n * _LN2_HI).astype(np.float32)).astype(np.float32)
        r = (r - (n * _LN2_LO).astype(np.float32)).astype(np.float32)
        p = np.full_like(r, _TAYLOR[0])
        for c in _TAYLOR[1:]:
            p = ((p * r).astype(np.float32) + c).astype(np.float32)
        scale = ((n.astype(np.int64) + 127).astype(np.uint32) << np.uint32(23)).view(np.float32)
        out = (p * scale).astype(np.float32)
    return np.where(low, F(0.0), out).astype(np.float32)


def sort_key(x: np.ndarray) -> np.ndarray:
    u = np.asarray(x, dtype=np.float32).view(np.uint32)
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def wave_scan(w: np.ndarray) -> np.ndarray:
    """Inclusive cumulative sums of w (float32, rank order) as the kernel forms them.

    Lane L of 64 owns ranks [L*E, L*E+E) with E = ceil(k/64); inside a lane
    the sums run sequentially; the lane totals go through a Kogge-Stone
    inclusive scan (step d: S_L <- S_L + S_{L-d} for L >= d, all lanes at
    once); cum_r = S_{L-1} + local_r (S_{-1} = 0).
    """

    w = np.asarray(w, dtype=np.float32)
    k = len(w)
    e = -(-k // 64)
    local = np.zeros(k, dtype=np.float32)
    totals = np.zeros(64, dtype=np.float32)
    for lane in range(64):
        acc = F(0.0)
        for r in range(lane * e, min(k, lane * e + e)):
            acc = F(acc + w[r])
            local[r] = acc
        totals[lane] = acc
    s = totals.copy()
    d = 1
    while d < 64:
        prev = s.copy()
        s[d:] = (prev[d:] + prev[:-d]).astype(np.float32)
        d <<= 1
    excl = np.concatenate(([F(0.0)], s[:-1])).astype(np.float32)
    cum = np.empty(k, dtype=np.float32)
    for lane in range(64):
        for r in range(lane * e, min(k, lane * e + e)):
            cum[r] = F(excl[lane] + local[r])
    return cum


def prepare(logits: np.ndarray, penalty: float, seen: np.ndarray | None, mask_from: int, eos_id: int,
            suppress_eos: bool) -> np.ndarray:
    x = np.asarray(logits, dtype=np.float32).copy()
    v = x.shape[0]
    ids = np.arange(v)
    masked = ((ids >= mask_from) & (ids != eos_id)) | ((ids == eos_id) & bool(suppress_eos))
    x[masked] = -np.inf
    if seen is not None:
        r = F(penalty)
        with np.errstate(invalid="ignore"):
            pen = np.where(x > 0, (x / r).astype(np.float32), (x * r).astype(np.float32))
        x = np.where(seen.astype(bool), pen, x).astype(np.float32)
    return x


def sample_row(logits: np.ndarray, temperature: float, top_k: int, top_p: float, u: float,
               penalty: float = 1.0, seen: np.ndarray | None = None, mask_from: int | None = None,
               eos_id: int = -1, suppress_eos: bool = False) -> int:
    v = logits.shape[0]
    x = prepare(logits, penalty, seen, v if mask_from is None else mask_from, eos_id, suppress_eos)
    t = F(temperature)
    if t == 0:
        keys = sort_key(x).astype(np.uint64)
        comp = (keys << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - np.arange(v, dtype=np.uint64))
        return 0xFFFFFFFF - (int(comp.max()) & 0xFFFFFFFF)
    s = (x / t).astype(np.float32)
    k_eff = int(top_k) if 0 < int(top_k) < v else v
    p = min(F(top_p), F(1.0))
    keys = sort_key(s).astype(np.uint64)
    comp = (keys << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - np.arange(v, dtype=np.uint64))
    order = np.argsort(comp, kind="stable")[::-1][:k_eff]
    vals = s[order]
    v0 = vals[0]
    if v0 == -np.inf:
        return int(order[0])
    w = nq_exp((vals - v0).astype(np.float32))
    cum = wave_scan(w)
    total = cum[k_eff - 1]
    pt = F(p * total)
    drop = np.nonzero(~((cum - w).astype(np.float32) < pt))[0]
    kept = int(drop[0]) if len(drop) else k_eff
    kept = max(kept, 1)
    mass = cum[kept - 1]
    um = F(F(u) * mass)
    hit = np.nonzero(cum[:kept] >= um)[0]
    pick = int(hit[0]) if len(hit) else kept - 1
    return int(order[pick])


def sample(logits, temperature, top_k, top_p, uniforms, penalty=None, seen=None, mask_from=None,
           eos_id=-1, suppress_eos=None) -> np.ndarray:
    """Batch form of ``sample_row``; every argument is per row."""

    logits = np.asarray(logits, dtype=np.float32)
    rows = logits.shape[0]
    out = np.empty(rows, dtype=np.int64)
    for r in range(rows):
        out[r] = sample_row(
            logits[r],
            float(temperature[r]),
            int(top_k[r]),
            float(top_p[r]),
            float(uniforms[r]),
            1.0 if penalty is None else float(penalty[r]),
            None if seen is None else seen[r],
            mask_from,
            eos_id,
            False if suppress_eos is None else bool(suppress_eos[r]),
        )
    return out


# --- Philox-4x32-10 -------------------------------------------------------

_M0, _M1 = 0xD2511F53, 0xCD9E8D57
_W0, _W1 = 0x9E3779B9, 0xBB67AE85
_MASK = 0xFFFFFFFF


def philox4x32(counter: tuple[int, int, int, int], key: tuple[int, int], rounds: int = 10):
    c0, c1, c2, c3 = (int(x) & _MASK for x in counter)
    k0, k1 = (int(x) & _MASK for x in key)
    for _ in range(rounds):
        p0 = _M0 * c0
        p1 = _M1 * c2
        c0, c1, c2, c3 = ((p1 >> 32) ^ c1 ^ k0) & _MASK, p1 & _MASK, ((p0 >> 32) ^ c3 ^ k1) & _MASK, p0 & _MASK
        k0 = (k0 + _W0) & _MASK
        k1 = (k1 + _W1) & _MASK
    return c0, c1, c2, c3


def uniform_from_counter(seed: int, offset: int) -> np.float32:
    s = int(seed) & 0xFFFFFFFFFFFFFFFF
    o = int(offset) & 0xFFFFFFFFFFFFFFFF
    x0 = philox4x32((o & _MASK, o >> 32, 0, 0), (s & _MASK, s >> 32))[0]
    return F(x0 >> 8) * F(1.0 / 16777216.0)
