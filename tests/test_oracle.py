"""Pins the CPU oracle (oracle/) without trusting its own formulas: against a library routine
(torch's scaled_dot_product_attention), brute-force loops on tiny inputs, and closed-form
invariants chosen so that a dropped term, a sign or index error or a transposed operand fails.
The reference ships no golden vectors for this path (its tests read model dumps that are not in
the repository), so these checks are what fix the oracle; tests/golden/ holds fixtures made by
the pinned oracle for the GPU tests to reuse."""

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as O
from oracle import planner as OP


def rnd(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


def brute_decode(q, k, v, scale, keep=None):
    """Pure-Python loops: softmax attention of each query head over its KV head's kept tokens."""
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = torch.zeros(B, Hq, D, dtype=torch.float64)
    lse = torch.full((B, Hq), -math.inf, dtype=torch.float64)
    for b in range(B):
        for h in range(Hq):
            kh = h // G
            toks = [t for t in range(T) if keep is None or bool(keep[b, kh, t // 64])]
            if not toks:
                continue
            s = [scale * sum(float(q[b, h, d]) * float(k[b, kh, t, d]) for d in range(D)) for t in toks]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            lse[b, h] = m + math.log(z)
            for d in range(D):
                out[b, h, d] = sum(wi * float(v[b, kh, t, d]) for wi, t in zip(w, toks)) / z
    return out, lse


def test_decode_vs_sdpa():
    for (B, Hq, Hkv, T, D) in ((2, 8, 2, 300, 16), (1, 28, 4, 129, 32), (3, 4, 4, 64, 8)):
        q, k, v = rnd(B, Hq, D, seed=1), rnd(B, Hkv, T, D, seed=2), rnd(B, Hkv, T, D, seed=3)
        out, lse = O.decode(q, k, v, 0.37)
        ref = F.scaled_dot_product_attention(q[:, :, None], k, v, scale=0.37, enable_gqa=True)[:, :, 0]
        assert torch.allclose(out, ref, atol=1e-12, rtol=1e-10)
        s = torch.einsum("bhd,bhtd->bht", q, k.repeat_interleave(Hq // Hkv, 1)) * 0.37
        assert torch.allclose(lse, torch.logsumexp(s, -1), atol=1e-12)


def test_decode_masked_vs_brute_and_gather():
    B, Hq, Hkv, T, D = 2, 4, 2, 150, 3
    q, k, v = rnd(B, Hq, D, seed=4), rnd(B, Hkv, T, D, seed=5), rnd(B, Hkv, T, D, seed=6)
    keep = torch.tensor([[[1, 0, 1], [0, 1, 0]], [[0, 0, 1], [1, 1, 1]]], dtype=torch.bool)
    out, lse = O.decode(q, k, v, 0.5, keep=keep)
    bo, bl = brute_decode(q, k, v, 0.5, keep)
    assert torch.allclose(out, bo, atol=1e-12) and torch.allclose(lse, bl, atol=1e-12)
    # masked == SDPA on the gathered kept tokens, per (b, kv head)
    for b in range(B):
        for h in range(Hkv):
            toks = torch.nonzero(O.token_mask(keep[b, h], T)).flatten()
            ref = F.scaled_dot_product_attention(q[b:b + 1, 2 * h:2 * h + 2, None], k[b:b + 1, h:h + 1, toks],
                                                 v[b:b + 1, h:h + 1, toks], scale=0.5)[0, :, 0]
            assert torch.allclose(out[b, 2 * h:2 * h + 2], ref, atol=1e-12)
    # empty kept set: out 0, lse -inf (what a kernel that reads nothing returns)
    out, lse = O.decode(q, k, v, 0.5, keep=torch.zeros_like(keep))
    assert (out == 0).all() and torch.isinf(lse).all()


def test_block_stats_invariants():
    B, Hq, Hkv, T, D = 1, 6, 3, 200, 8
    q, k = rnd(B, Hq, D, seed=7), rnd(B, Hkv, T, D, seed=8)
    M, S = O.block_stats(q, k, 0.3)
    s = O.scores(q, k, 0.3)
    # the block log-weights merge to the full log-sum-exp; each block max is attained
    assert torch.allclose(torch.logsumexp(O.block_logw(M, S), -1), torch.logsumexp(s, -1), atol=1e-12)
    for blk in range(O.nblocks(T)):
        seg = s[..., blk * 64:min(T, blk * 64 + 64)]
        assert torch.equal(M[..., blk], seg.amax(-1))
        assert torch.allclose(S[..., blk], torch.exp(seg - seg.amax(-1, keepdim=True)).sum(-1), atol=1e-12)
    # P: exp(s - block max) reproduces exp(s) after scaling back, 1 at the block max, 0 past T
    P = O.p_values(q, k, 0.3)
    assert torch.allclose(P[..., :T] * torch.exp(M.repeat_interleave(64, -1)[..., :T]), torch.exp(s), rtol=1e-12)
    assert (P[..., T:] == 0).all() and torch.allclose(P.reshape(B, Hq, -1, 64).amax(-1), torch.ones_like(M))
    keep = torch.zeros(B, Hkv, O.nblocks(T), dtype=torch.bool)
    keep[..., 1] = True
    Mk, Sk = O.block_stats(q, k, 0.3, keep=keep)
    assert torch.isinf(Mk[..., 0]).all() and (Sk[..., 0] == 0).all() and torch.equal(Mk[..., 1], M[..., 1])


def brute_topp(w, level):
    """Fewest blocks whose weights reach `level` (all subsets); ties at the cut kept."""
    n = len(w)
    for size in range(1, n + 1):
        best = max(itertools.combinations(range(n), size), key=lambda c: sum(w[i] for i in c))
        if sum(w[i] for i in best) >= level:
            thr = min(w[i] for i in best)
            return {i for i in range(n) if w[i] >= thr}
    return set(range(n))


def test_topp_vs_brute_force():
    g = torch.Generator().manual_seed(9)
    for trial in range(200):
        nb = int(torch.randint(1, 9, (1,), generator=g))
        logw = torch.randn(1, 1, nb, generator=g, dtype=torch.float64) * 3
        level = float(torch.rand((), generator=g)) * 0.5 + 0.5
        keep_h, _ = O.topp_heads(logw, level)
        w = torch.softmax(logw[0, 0], -1).tolist()
        assert set(torch.nonzero(keep_h[0, 0]).flatten().tolist()) == brute_topp(w, level), (logw, level)
    # GQA union + sink + local, rule tau
    logw = rnd(1, 4, 10, seed=10) * 2
    keep = O.select_blocks(logw, 2, "tau", 0.1, local=2)
    W = torch.softmax(logw, -1)
    for h in range(2):
        for blk in range(10):
            expect = blk == 0 or blk >= 8 or bool((W[0, 2 * h:2 * h + 2, blk] >= 0.1).any())
            assert bool(keep[0, h, blk]) == expect


def test_vskip1_rule_vs_brute():
    B, Hq, Hkv, T, D = 1, 4, 2, 64 * 6 + 5, 4
    q, k = rnd(B, Hq, D, seed=11) * 2, rnd(B, Hkv, T, D, seed=12)
    for lp in (None, torch.tensor([[3.0, 4.0, 5.0, 6.0]], dtype=torch.float64)):
        keep, z = O.vskip1_keep(q, k, 0.5, 1e-2, 1, lse_prev=lp)
        s = O.scores(q, k, 0.5)
        for h in range(Hkv):
            for blk in range(7):
                lse_b = [float(torch.logsumexp(s[0, g, blk * 64:min(T, blk * 64 + 64)], -1)) for g in (2 * h, 2 * h + 1)]
                lse0 = [float(torch.logsumexp(s[0, g, :64], -1)) if lp is None else float(lp[0, g]) for g in (2 * h, 2 * h + 1)]
                vote = any(a - b >= math.log(1e-2) for a, b in zip(lse_b, lse0))
                assert bool(keep[0, h, blk]) == (blk == 0 or blk == 6 or vote)


def test_two_pass_identity():
    """pass 2 with blk_scale = exp(blk_max - lse_kept) on the pass-1 P is exact attention over the
    kept set (kernels/kvskip.py:157-179)."""
    B, Hq, Hkv, T, D = 1, 4, 2, 300, 8
    q, k, v = rnd(B, Hq, D, seed=13), rnd(B, Hkv, T, D, seed=14), rnd(B, Hkv, T, D, seed=15)
    M, S = O.block_stats(q, k, 0.4)
    logw = O.block_logw(M, S)
    keep = O.select_blocks(logw, 2, "topp", 0.9, local=1)
    kh = O.heads(keep, 2)
    lse_kept = logw.masked_fill(~kh, -math.inf).logsumexp(-1, keepdim=True)
    scale_b = torch.exp(M - lse_kept).masked_fill(~kh, 0.0).reshape(B, Hkv, 2, -1).transpose(2, 3)
    out = O.pv(O.p_values(q, k, 0.4), v, scale_b, keep)
    ref, _ = O.decode(q, k, v, 0.4, keep=keep)
    assert torch.allclose(out, ref, atol=1e-12)


def test_split_ranges():
    for n in (0, 1, 7, 64, 65):
        for S in (1, 3, 8, 70):
            r = O.split_ranges(n, S)
            assert len(r) == S and r[0][0] == 0 and r[-1][1] == n
            assert all(a[1] == b[0] for a, b in zip(r, r[1:]))


def test_centroids_vs_loops():
    B, Hq, Hkv, T, D = 1, 4, 2, 130, 3
    q, k = rnd(B, Hq, D, seed=16), rnd(B, Hkv, T, D, seed=17)
    cs = OP.centroid_sums(k)
    sc = OP.centroid_scores(q, cs, T, 0.7)
    for h in range(Hq):
        for blk in range(3):
            rows = range(blk * 64, min(T, blk * 64 + 64))
            c = [sum(float(k[0, h // 2, t, d]) for t in rows) / len(rows) for d in range(D)]
            assert abs(float(sc[0, h, blk]) - 0.7 * sum(float(q[0, h, d]) * c[d] for d in range(D))) < 1e-12


def _layer(T=2000, G=4, Hkv=2, D=16, seed=18):
    q = rnd(1, G * Hkv, D, seed=seed) * 1.5
    k = rnd(1, Hkv, T, D, seed=seed + 1)
    k[:, :, 0:64] += 2.0 * q.reshape(1, Hkv, G, D).mean(2)[:, :, None] / D ** 0.5
    return q, k, rnd(1, Hkv, T, D, seed=seed + 2)


def test_estimate_is_exact_at_refresh():
    """Right after a refresh, with the same query and no new token, every centroid score equals its
    reference, so the estimate is the block log-sum-exp over the blocks outside the attended set:
    miss = that set's true missed softmax mass (brute force), which top-p 0.99 keeps <= 0.01."""
    q, k, v = _layer()
    pol = OP.Policy(level=0.99)
    st, _ = OP.init(q, k, v, 1.0, pol)
    pr = OP.plan(st, q, k, pol)
    p = torch.softmax(O.scores(q, k, 1.0), -1)                                      # [1, Hq, T]
    att = O.heads(O.token_mask(st.keep | O.always_keep(O.nblocks(k.shape[2]), pol.local), k.shape[2]), 4)
    missed = (p * ~att).sum(-1).reshape(1, 2, 4).amax(-1)
    assert torch.allclose(pr["miss"], missed, atol=1e-12)
    assert (missed > 0).all() and (missed <= 1 - pol.level + 1e-12).all() and not pr["trig"].any()
    assert not st.keep.all()


def test_estimate_tracks_drift_and_triggers():
    """Moving the query onto keys outside the stored set raises the estimate past delta (refresh);
    the age limit and forced heads refresh regardless; the warm-up shortens the age limit."""
    q, k, v = _layer(seed=30)
    pol = OP.Policy(delta=0.05, max_age=3, dense_heads=(1,))
    st, _ = OP.init(q, k, v, 1.0, pol)
    # query head 0 turns to the mean key of a block outside its group's stored set
    outside = int(torch.nonzero(~(st.keep[0, 0] | O.always_keep(st.keep.shape[-1], 2)))[0])
    c = k[0, 0, outside * 64:outside * 64 + 64].mean(0)
    q2 = q.clone()
    q2[0, 0] = 40.0 * c / c.norm()
    pr = OP.plan(st, q2, k, pol)
    assert bool(pr["trig"][0, 0]) and pr["dec"][0, 0] > pol.delta and bool(pr["trig"][0, 1])
    assert bool(pr["read"][0, 0].all())
    # the unchanged query of the same state does not trigger; the age limit then does
    st, _ = OP.init(q, k, v, 1.0, pol)
    for t in range(1, 4):
        pr = OP.plan(st, q, k, pol)
        assert bool(pr["trig"][0, 0]) == (t == 3) and bool(pr["trig"][0, 1])
    warm = OP.Policy(max_age=3, calib_warm=(2, 1))
    assert OP.max_age_at(warm, 1) == 1 and OP.max_age_at(warm, 2) == 3


def test_calibration_peak_bounds_the_residual():
    """kind "peak" keeps c >= real - estimate on every refresh (decaying maximum); with rate 0 it is
    exactly the largest residual seen; real = the attended set's true missed mass."""
    q, k, v = _layer(seed=40)
    pol = OP.Policy(calib=0.0, calib_kind="peak", dense_heads=(0, 1))
    st, _ = OP.init(q, k, v, 1.0, pol)
    q2 = q + 0.8 * rnd(*q.shape, seed=41)
    out, pr = OP.step(st, q2, k, v, pol)
    assert (pr["miss"] > 0).all()
    p = torch.softmax(O.scores(q2, k, 1.0), -1)
    att = O.heads(O.token_mask(pr["sel"], k.shape[2]), 4)
    real = (p * ~att).sum(-1).reshape(1, 2, 4).amax(-1)
    assert (real > 0).all()
    assert torch.allclose(st.calib, torch.clamp(real - pr["miss"], min=0.0), atol=1e-12)


@pytest.mark.parametrize("kind", ["add", "logit"])
def test_calibration_ema_kinds_closed_form(kind):
    """Kinds "add" and "logit" are exponential averages of the residual; at rate 1 the new c is the
    residual itself (real - est, or logit(real) - logit(est) with the 1e-6 clamp), at rate 0 the old
    c, and in between their convex mix (rate 0.3, starting from c = 0.2); clamped at 0 unless free."""
    q, k, v = _layer(seed=42)
    q2 = q + 0.8 * rnd(*q.shape, seed=43)
    p = torch.softmax(O.scores(q2, k, 1.0), -1)

    def run(rate, c0, free=False):
        pol = OP.Policy(calib=rate, calib_kind=kind, dense_heads=(0, 1), calib_free=free)
        st, _ = OP.init(q, k, v, 1.0, pol)
        st.calib = torch.full_like(st.calib, c0)
        _, pr = OP.step(st, q2, k, v, pol)
        att = O.heads(O.token_mask(pr["sel"], k.shape[2]), 4)
        real = (p * ~att).sum(-1).reshape(1, 2, 4).amax(-1)
        clamp = lambda x: x.clamp(1e-6, 1 - 1e-6)
        lg = lambda x: torch.log(clamp(x)) - torch.log1p(-clamp(x))
        resid = real - pr["miss"] if kind == "add" else lg(real) - lg(pr["miss"])
        return st.calib, resid

    c1, resid = run(1.0, 0.2, free=True)
    assert torch.allclose(c1, resid, atol=1e-12)
    c0, _ = run(0.0, 0.2)
    assert torch.allclose(c0, torch.full_like(c0, 0.2), atol=1e-15)
    cm, resid = run(0.3, 0.2)
    assert torch.allclose(cm, (0.7 * 0.2 + 0.3 * resid).clamp_min(0.0), atol=1e-12)


def test_token_index_vs_loops():
    g = np.random.default_rng(3)
    ids = g.integers(0, 7, size=(2, 300))
    for T in (1, 2, 64, 65, 200, 300):
        got = OP.index_blocks(ids, T)
        for b in range(2):
            cur = ids[b, T - 1]
            for blk in range(O.nblocks(T)):
                hit = False
                for j in range(blk * 64, min(T, blk * 64 + 64)):
                    same = j < T - 1 and ids[b, j] == cur
                    after = j >= 1 and j - 1 < T - 1 and ids[b, j - 1] == cur
                    hit = hit or same or after
                assert got[b, blk] == hit


def test_attended_lse_all_blocks_is_full_lse():
    q, k, v = _layer(seed=50)
    M, S = O.block_stats(q, k, 0.25)
    full = OP.attended_lse(O.block_logw(M, S), torch.ones(1, 2, M.shape[-1], dtype=torch.bool), 4)
    assert torch.allclose(full, torch.logsumexp(O.scores(q, k, 0.25), -1), atol=1e-12)


# ---------------------------------------------------------------- planner pieces pinned separately

def brute_index(ids, T):
    """Loops: blocks with an earlier copy of ids[T-1], or the position right after one."""
    cur = ids[T - 1]
    hits = set()
    for t in range(T):
        if (t < T - 1 and ids[t] == cur) or (1 <= t and t - 1 < T - 1 and ids[t - 1] == cur):
            hits.add(t // 64)
    return hits


def test_update_csum_appended_keys():
    """Key sums kept current by adding the appended rows (one at a time up to a full block, into a
    new block, several at once) equal the sums of the grown cache from scratch and by loops
    (src/kvskip_attn.py:273-279 against src/kvskip_attn.py:170-179)."""
    B, Hkv, D = 1, 2, 5
    k = rnd(B, Hkv, 330, D, seed=60)
    q, v = rnd(B, 4, D, seed=61), rnd(B, Hkv, 330, D, seed=62)
    st, _ = OP.init(q, k[:, :, :127], v[:, :, :127], 1.0, OP.Policy())
    for T in (128, 129, 130, 192, 193, 260, 330):
        OP.update_csum(st, k[:, :, :T])
        assert st.T == T and st.csum.shape == (B, Hkv, O.nblocks(T), D)
        assert torch.allclose(st.csum, OP.centroid_sums(k[:, :, :T]), atol=1e-12)
    for h in range(Hkv):
        for blk in range(O.nblocks(330)):
            for d in range(D):
                ref = sum(float(k[0, h, t, d]) for t in range(blk * 64, min(330, blk * 64 + 64)))
                assert abs(float(st.csum[0, h, blk, d]) - ref) < 1e-12
    # the plan's centroid scores then use the grown sums (partial last block: its own row count)
    st2, _ = OP.init(q, k[:, :, :200], v[:, :, :200], 1.0, OP.Policy())
    pr = OP.plan(st2, q, k[:, :, :201], OP.Policy())
    assert torch.allclose(pr["cs"], OP.centroid_scores(q, OP.centroid_sums(k[:, :, :201]), 201, 1.0), atol=1e-12)


def test_index_only_heads_read_the_index_and_never_refresh():
    """A token-index head reads index blocks + sink + local only and never refreshes, whatever its
    drift or age (src/kvskip_attn.py:381-383); the other heads refresh by age."""
    q, k, v = _layer(seed=70)
    T = k.shape[2]
    nb = O.nblocks(T)
    ids = np.random.default_rng(71).integers(0, 40, size=(1, T))
    idx = torch.from_numpy(OP.index_blocks(ids, T))
    hits = brute_index(ids[0], T)
    assert 0 < len(hits) < nb - 3
    pol = OP.Policy(max_age=2, index_heads=(1,), index_union=False)
    st, _ = OP.init(q, k, v, 1.0, pol)
    keep1 = st.keep[0, 1].clone()
    q2 = q.clone()
    outside = int(torch.nonzero(~(st.keep[0, 1] | O.always_keep(nb, 2)))[0])
    c = k[0, 1, outside * 64:outside * 64 + 64].mean(0)
    q2[0, 4:8] = 40.0 * c / c.norm()                # KV head 1's queries drift far outside its set
    for t in range(1, 5):
        out, pr = OP.step(st, q2, k, v, pol, idx=idx)
        assert not bool(pr["trig"][0, 1]) and math.isinf(float(pr["margin"][0, 1]))
        expect = hits | {0, nb - 2, nb - 1}
        assert set(torch.nonzero(pr["read"][0, 1]).flatten().tolist()) == expect
        assert bool(pr["trig"][0, 0]) == (t % 2 == 0)        # age limit 2 on the ordinary head
        assert torch.equal(st.keep[0, 1], keep1)               # never refreshed
        # its output is attention over exactly the index blocks + sink + local
        ref, _ = O.decode(q2, k, v, 1.0, keep=pr["read"])
        assert torch.allclose(out[0, 4:8], ref[0, 4:8], atol=1e-12)
    assert OP.flags_of(pol, 2) == [0, 2]


def test_index_union_heads_attend_and_estimate_with_the_index():
    """An index-union head attends stored set + sink + local + index blocks (src/kvskip_attn.py:359-360)
    and still refreshes normally. Its estimate leaves the index blocks out of the missed part: right
    after a refresh with the same query, miss = P_out / (P_out + P_att) by brute force, P_out the
    softmax mass outside that larger set and P_att the mass of the previous step's attended set
    (stored + sink + local, the lse_att of src/kvskip_attn.py:392)."""
    q, k, v = _layer(seed=72)
    T = k.shape[2]
    nb = O.nblocks(T)
    ids = np.random.default_rng(73).integers(0, 30, size=(1, T))
    idx = torch.from_numpy(OP.index_blocks(ids, T))
    pol = OP.Policy(index_heads=(1,), index_union=True)
    st, _ = OP.init(q, k, v, 1.0, pol)
    stored = st.keep.clone()
    pr = OP.plan(st, q, k, pol, idx=idx)
    always = O.always_keep(nb, 2)
    assert torch.equal(pr["sel"][0, 0], stored[0, 0] | always)
    assert torch.equal(pr["sel"][0, 1], stored[0, 1] | always | idx[0])
    assert bool((idx[0] & ~(stored[0, 1] | always)).any())          # the index adds blocks
    p = torch.softmax(O.scores(q, k, 1.0), -1)
    p_out = (p * ~O.heads(O.token_mask(pr["sel"], T), 4)).sum(-1)
    p_att = (p * O.heads(O.token_mask(stored | always, T), 4)).sum(-1)
    missed = (p_out / (p_out + p_att)).reshape(1, 2, 4).amax(-1)
    assert torch.allclose(pr["miss"], missed, atol=1e-12)
    plain = (p * ~O.heads(O.token_mask(stored | always, T), 4)).sum(-1).reshape(1, 2, 4)[0, 1].amax()
    assert float(missed[0, 1]) < float(plain)                             # the index blocks are not missed
    pol_dense = OP.Policy(index_heads=(1,), index_union=True, dense_heads=(1,))
    st, _ = OP.init(q, k, v, 1.0, pol_dense)
    assert bool(OP.plan(st, q, k, pol_dense, idx=idx)["trig"][0, 1])   # a forced union head refreshes
    assert OP.flags_of(pol_dense, 2) == [0, 5]


def test_auto_index_latch_threshold_and_union():
    """The latch: after each step's calibration every head with correction > threshold joins the
    token index for good (src/kvskip_attn.py:318-319), strictly above, sticky, refreshing or not;
    a latched head's attended set then includes the index blocks (src/kvskip_attn.py:361-362)."""
    q, k, v = _layer(seed=74)
    T = k.shape[2]
    nb = O.nblocks(T)
    ids = np.random.default_rng(75).integers(0, 30, size=(1, T))
    idx = torch.from_numpy(OP.index_blocks(ids, T))
    thr = 0.25
    # rate 0: c = max(c, resid); delta 0.9 keeps miss + c under it (no refresh)
    pol = OP.Policy(delta=0.9, calib=0.0, calib_kind="peak", calib_auto_ix=thr)
    st, _ = OP.init(q, k, v, 1.0, pol)
    up = math.nextafter(thr, math.inf)
    st.calib = torch.tensor([[thr, up]], dtype=torch.float64)           # equal: no latch; above: latch
    _, pr = OP.step(st, q, k, v, pol, idx=idx)
    assert not pr["trig"].any()                                         # no head refreshed
    assert st.aix.tolist() == [[False, True]]
    stored = st.keep.clone()
    st.calib = torch.zeros_like(st.calib)                               # below the threshold: stays latched
    pr = OP.plan(st, q, k, pol, idx=idx)
    assert st.aix.tolist() == [[False, True]]
    always = O.always_keep(nb, 2)
    assert torch.equal(pr["sel"][0, 0], stored[0, 0] | always)
    assert torch.equal(pr["sel"][0, 1], stored[0, 1] | always | idx[0])
    # a threshold below the initial correction latches every head on the first step
    pol_neg = OP.Policy(calib=0.05, calib_kind="peak", calib_auto_ix=-1.0)
    st, _ = OP.init(q, k, v, 1.0, pol_neg)
    OP.step(st, q, k, v, pol_neg, idx=idx)
    assert st.aix.all()


def test_flags_of():
    """Bit 0: refreshed on every step; bit 1: token-index head; bit 2: index union; OR-ed per head
    (src/kvskip_attn.py:413-419)."""
    assert OP.flags_of(OP.Policy(), 3) == [0, 0, 0]
    assert OP.flags_of(OP.Policy(dense_heads=(0, 2)), 3) == [1, 0, 1]
    assert OP.flags_of(OP.Policy(index_heads=(1,)), 3) == [0, 2, 0]
    assert OP.flags_of(OP.Policy(index_heads=(1, 2), index_union=True), 3) == [0, 4, 4]
    assert OP.flags_of(OP.Policy(dense_heads=(1,), index_heads=(1,)), 2) == [0, 3]
    # a head in both lists with index-only: the index rule wins (no refresh), as in refresh_pre
    q, k, v = _layer(seed=76)
    ids = np.random.default_rng(77).integers(0, 30, size=(1, k.shape[2]))
    idx = torch.from_numpy(OP.index_blocks(ids, k.shape[2]))
    pol = OP.Policy(dense_heads=(1,), index_heads=(1,))
    st, _ = OP.init(q, k, v, 1.0, pol)
    assert not bool(OP.plan(st, q, k, pol, idx=idx)["trig"][0, 1])


def test_topp_margin_per_head():
    """update() records each refreshed query head's own top-p margin (inf for the others)."""
    q, k, v = _layer(seed=78)
    pol = OP.Policy(dense_heads=(0,))
    st, _ = OP.init(q, k, v, 1.0, pol)
    _, pr = OP.step(st, q, k, v, pol)
    M, S = O.block_stats(q, k, 1.0, keep=pr["read"])
    _, margin = O.topp_heads(O.block_logw(M, S), pol.level)
    assert torch.equal(st.topp_heads[0, :4], margin[0, :4]) and torch.isinf(st.topp_heads[0, 4:]).all()


# ---------------------------------------------------------------- the "refresh" mode (post trigger)

def _brute_block_lse(q, k, scale, T):
    """Per query head and block: log-sum-exp of the block's scores, block by block with explicit dot
    products: [B, Hq, nb]."""
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    nb = O.nblocks(T)
    out = torch.empty(B, Hq, nb, dtype=torch.float64)
    for b in range(B):
        for h in range(Hq):
            for blk in range(nb):
                rows = k[b, h // G, blk * 64:min(T, blk * 64 + 64)]
                out[b, h, blk] = torch.logsumexp(scale * (rows @ q[b, h]), 0)
    return out


def _brute_centroid_scores(q, k, scale, T):
    B, Hq, D = q.shape
    G = Hq // k.shape[1]
    nb = O.nblocks(T)
    out = torch.empty(B, Hq, nb, dtype=torch.float64)
    for b in range(B):
        for h in range(Hq):
            for blk in range(nb):
                c = k[b, h // G, blk * 64:min(T, blk * 64 + 64)].mean(0)
                out[b, h, blk] = scale * float(q[b, h] @ c)
    return out


def _post_case(seed):
    """A layer of 700 tokens (init at fewer, then appended ones) and a drifted query."""
    q, k, v = _layer(T=700, D=8, seed=seed)
    q2 = q + 0.6 * rnd(*q.shape, seed=seed + 7)
    return q, q2, k, v


def _post_reference(q, q2, k, v, scale, keep0, local):
    """Brute-force decision inputs of the step after the refresh at T0 = T - 1: the attended set,
    its log-sum-exp under THIS step's query, and per KV head the missed-mass estimate
    sigma(lse(est over the unattended blocks) - lse_sel) maxed over the group, with
    est_b = lse_ref_b + cs_b(q2, T) - cs_ref_b (references from q at T0)."""
    T = k.shape[2]
    G = q.shape[1] // k.shape[1]
    nb = O.nblocks(T)
    sel = OP.pad_blocks(keep0, nb, False) | O.always_keep(nb, local)
    lse_ref = _brute_block_lse(q, k[:, :, :T - 1], scale, T - 1)
    cs_ref = _brute_centroid_scores(q, k[:, :, :T - 1], scale, T - 1)
    cs_now = _brute_centroid_scores(q2, k, scale, T)
    _, lse_sel = brute_decode(q2, k, v, scale, keep=sel)
    _, lse_old = brute_decode(q, k[:, :, :T - 1], v[:, :, :T - 1], scale, keep=sel)   # the previous step's
    B, Hq = lse_sel.shape
    miss = torch.zeros(B, Hq // G, dtype=torch.float64)
    miss_old = torch.zeros_like(miss)
    for b in range(B):
        for h in range(Hq):
            est = [float(lse_ref[b, h, i] + cs_now[b, h, i] - cs_ref[b, h, i])
                   for i in range(nb) if not bool(sel[b, h // G, i])]
            if not est:
                continue
            e = torch.logsumexp(torch.tensor(est, dtype=torch.float64), 0)
            miss[b, h // G] = max(float(miss[b, h // G]), float(torch.sigmoid(e - lse_sel[b, h])))
            miss_old[b, h // G] = max(float(miss_old[b, h // G]), float(torch.sigmoid(e - lse_old[b, h])))
    return sel, miss, miss_old, cs_now


def test_post_step_decides_on_this_steps_lse():
    """The refresh mode's estimate (src/kvskip_attn.py:241-251) against brute force, with the
    log-sum-exp of this step's masked pass; the previous step's (refresh_pre's) gives a clearly
    different number here, so the test tells them apart. delta set between the two KV heads'
    estimates: one refreshes (dense output, new set from its full statistics, age 0), the other keeps
    its masked output (brute-force masked attention), set and age + 1."""
    scale = 3.0
    q, q2, k, v = _post_case(80)
    T = k.shape[2]
    pol = OP.Policy(delta=0.05, max_age=32)
    st0, _ = OP.init(q, k[:, :, :T - 1], v[:, :, :T - 1], scale, pol)
    sel, miss, miss_old, cs_now = _post_reference(q, q2, k, v, scale, st0.keep, pol.local)
    assert (miss > 0).all() and (miss - miss_old).abs().min() > 1e-3
    lo, hi = sorted(miss[0].tolist())
    assert hi - lo > 1e-3
    pol = OP.Policy(delta=(lo + hi) / 2, max_age=32)
    st, _ = OP.init(q, k[:, :, :T - 1], v[:, :, :T - 1], scale, pol)
    keep0 = st.keep.clone()
    out, pr = OP.post_step(st, q2, k, v, pol)
    assert torch.allclose(pr["miss"], miss, atol=1e-10)
    assert torch.equal(pr["sel"], sel)
    trig = miss > pol.delta
    assert torch.equal(pr["trig"], trig) and int(trig.sum()) == 1
    dense = F.scaled_dot_product_attention(q2[:, :, None], k, v, scale=scale, enable_gqa=True)[:, :, 0]
    masked, _ = brute_decode(q2, k, v, scale, keep=sel)
    G = 4
    for h in range(2):
        ref = dense if bool(trig[0, h]) else masked
        assert torch.allclose(out[:, h * G:(h + 1) * G], ref[:, h * G:(h + 1) * G], atol=1e-10)
    # state: the refreshing head's set from its full statistics under q2 (top-p 0.99 union, brute
    # force), references = this step's block log-sum-exps and centroid scores; the other unchanged
    h_t, h_k = (0, 1) if bool(trig[0, 0]) else (1, 0)
    lse_now = _brute_block_lse(q2, k, scale, T)
    nb = O.nblocks(T)
    kept = set()
    for g in range(G):
        w = torch.softmax(lse_now[0, h_t * G + g], -1).tolist()
        kept |= brute_topp(w, pol.level)
    kept |= {0} | set(range(nb - pol.local, nb))
    assert set(torch.nonzero(st.keep[0, h_t]).flatten().tolist()) == kept
    assert torch.equal(st.keep[0, h_k], OP.pad_blocks(keep0, nb, False)[0, h_k])
    rows = slice(h_t * G, (h_t + 1) * G)
    assert torch.allclose(st.lse_ref[0, rows], lse_now[0, rows], atol=1e-10)
    assert torch.allclose(st.cs_ref[0, rows], cs_now[0, rows], atol=1e-10)
    assert int(st.age[0, h_t]) == 0 and int(st.age[0, h_k]) == 1


def test_post_step_age_and_forced_heads():
    """max_age 1: every head refreshes on every step and the output is dense attention (SDPA);
    delta 1 with a forced head: only that head refreshes, the other keeps its set and its masked
    output (brute force) over the steps, its age counting up."""
    scale = 3.0
    q, q2, k, v = _post_case(80)
    T = k.shape[2]
    pol = OP.Policy(max_age=1)
    st, _ = OP.init(q, k[:, :, :T - 4], v[:, :, :T - 4], scale, pol)
    for t in range(T - 3, T + 1):
        out, pr = OP.post_step(st, q2, k[:, :, :t], v[:, :, :t], pol)
        ref = F.scaled_dot_product_attention(q2[:, :, None], k[:, :, :t], v[:, :, :t], scale=scale,
                                             enable_gqa=True)[:, :, 0]
        assert pr["trig"].all() and torch.allclose(out, ref, atol=1e-10)
    pol = OP.Policy(delta=1.0, max_age=1000, dense_heads=(1,))
    st, _ = OP.init(q, k[:, :, :T - 4], v[:, :, :T - 4], scale, pol)
    keep0 = st.keep[0, 0].clone()
    assert not keep0.all()
    for i, t in enumerate(range(T - 3, T + 1)):
        out, pr = OP.post_step(st, q2, k[:, :, :t], v[:, :, :t], pol)
        assert pr["trig"].tolist() == [[False, True]]
        nb = O.nblocks(t)
        sel = OP.pad_blocks(keep0[None, None], nb, False)[0, 0] | O.always_keep(nb, 2)
        assert torch.equal(pr["sel"][0, 0], sel) and int(st.age[0, 0]) == i + 1 and int(st.age[0, 1]) == 0
        masked, _ = brute_decode(q2[:, :4], k[:, :1, :t], v[:, :1, :t], scale, keep=sel[None, None])
        assert torch.allclose(out[:, :4], masked, atol=1e-10)
        ref = F.scaled_dot_product_attention(q2[:, 4:, None], k[:, 1:, :t], v[:, 1:, :t], scale=scale,
                                             enable_gqa=True)[:, :, 0]
        assert torch.allclose(out[:, 4:], ref, atol=1e-10)
