"""GPU parity of the attention kernels (through the C ABI, via kvskip_amd.ext) against the fp64
CPU oracle, on seeded inputs; the cases of the reference's bench/test_decode.py:66-196 plus the
BASELINE configurations.

Tolerances (bf16 in, fp32 accumulate): bf16 output rel. L2 error <= 2e-3 (the bar in the
north star; bf16 rounding of the output alone is ~1.1e-3), fp32 output <= 2e-5, lse and block
statistics (natural units) |err| <= 2e-4, block sums rel. <= 2e-4.
"""

import math

import pytest
import torch

from kvskip_amd import ext as E
from kvskip_amd import kvskip as K
from kvskip_amd import workloads as W
from oracle import attention as O

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-3
F32_TOL = 2e-5
LSE_TOL = 2e-4


def rand_qkv(B, Hq, Hkv, T, D, seed, sink_gap=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    if sink_gap:
        k[:, :, 0] *= 8.0                       # a sink with a ~30-nat gap (bench/test_decode.py:173)
    return q, k.to(torch.bfloat16), v


def to_gpu(*xs):
    return [x.cuda() for x in xs]


def check_decode(q, k, v, scale, gq, gk, gv, keep=None, num_splits=None, label=""):
    plan = None
    if keep is not None:
        plan = K.make_plan(keep.cuda())
    r = K.decode(gq, gk, gv, scale, plan=plan, num_splits=num_splits, out_f32=True)
    ref, lse = O.decode(q, k, v, scale, keep=keep)
    e16 = O.rel_err(r["out"].cpu(), ref)
    e32 = O.rel_err(r["out_f32"].cpu(), ref)
    el = (r["lse"].cpu().double() - lse).abs().max().item()
    print(f"{label} splits={r['num_splits']}: bf16 {e16:.2e} f32 {e32:.2e} lse {el:.2e}", flush=True)
    assert e16 <= BF16_TOL and e32 <= F32_TOL and el <= LSE_TOL, (label, e16, e32, el)
    return r


def test_cfg1_dense(gpu):
    L = W.cfg1()
    gq, gk, gv = to_gpu(L.q, L.k, L.v)
    for ns in (None, 1, 7, 64):
        check_decode(L.q, L.k, L.v, L.scale, gq, gk, gv, num_splits=ns, label="cfg1")


@pytest.mark.parametrize("D,T,ns", [(64, 1000, None), (64, 33, 3), (128, 64, 4), (128, 65, 9), (128, 3000, 64)])
def test_edge_cases(gpu, D, T, ns):
    """bench/test_decode.py:168-176: short / ragged T, more splits than blocks, huge score gaps."""
    q, k, v = rand_qkv(2, 32, 8, T, D, seed=T + D, sink_gap=True)
    check_decode(q, k, v, D ** -0.5, *to_gpu(q, k, v), num_splits=ns, label=f"D{D} T{T}")


@pytest.mark.parametrize("G", [1, 2, 4, 7, 8])
@pytest.mark.parametrize("D", [64, 128])
def test_group_sizes(gpu, G, D):
    q, k, v = rand_qkv(2, 4 * G, 4, 777, D, seed=10 * G + D)
    check_decode(q, k, v, D ** -0.5, *to_gpu(q, k, v), label=f"G{G} D{D}")
    keep = W.random_block_list(2, 4, O.nblocks(777), 0.4, seed=G)
    check_decode(q, k, v, D ** -0.5, *to_gpu(q, k, v), keep=keep, num_splits=3, label=f"G{G} D{D} masked")


def test_strided_layouts(gpu):
    """FA2 memory layout [B, T, Hkv, D] seen as [B, Hkv, T, D] (bench/test_decode.py:90-93), a
    growing-cache view (token stride D, head stride capacity * D), and a batch of 12."""
    q, k, v = rand_qkv(3, 32, 8, 1500, 128, seed=5)
    gq, gk, gv = to_gpu(q, k, v)
    ks = gk.transpose(1, 2).contiguous().transpose(1, 2)
    vs = gv.transpose(1, 2).contiguous().transpose(1, 2)
    check_decode(q, k, v, 128 ** -0.5, gq, ks, vs, label="bshd")
    cap = torch.zeros(3, 8, 2048, 128, dtype=torch.bfloat16, device="cuda")
    cap2 = torch.zeros_like(cap)
    cap[:, :, :1500] = gk
    cap2[:, :, :1500] = gv
    check_decode(q, k, v, 128 ** -0.5, gq, cap[:, :, :1500], cap2[:, :, :1500], label="capacity view")
    q, k, v = rand_qkv(12, 32, 8, 700, 128, seed=6)
    check_decode(q, k, v, 128 ** -0.5, *to_gpu(q, k, v), label="batch12")


def test_stats_and_stats_only(gpu):
    q, k, v = rand_qkv(2, 32, 8, 2000, 128, seed=7, sink_gap=True)
    gq, gk, gv = to_gpu(q, k, v)
    scale = 128 ** -0.5
    r = K.decode(gq, gk, gv, scale, stats=True, num_splits=5)
    M, S = O.block_stats(q, k, scale)
    fin = torch.isfinite(M)
    em = (r["blk_max"].cpu().double() - M)[fin].abs().max().item()
    es = ((r["blk_sum"].cpu().double() - S) / S)[fin].abs().max().item()
    lw = (O.block_logw(r["blk_max"].cpu().double(), r["blk_sum"].cpu().double()) - O.block_logw(M, S)).abs().max().item()
    print(f"stats: max |d blk_max| {em:.2e}, rel d blk_sum {es:.2e}, |d block lse| {lw:.2e}", flush=True)
    assert em <= LSE_TOL and es <= 2e-4 and lw <= LSE_TOL
    r2 = K.decode(gq, gk, gv, scale, stats=True, load_v=False)
    assert torch.equal(r2["blk_max"], r["blk_max"]) and torch.equal(r2["blk_sum"], r["blk_sum"]), \
        "stats-only differs from dense+stats"
    assert r2["out"] is None
    lse = torch.logsumexp(O.scores(q, k, scale), -1)
    assert (r2["lse"].cpu().double() - lse).abs().max().item() <= LSE_TOL


def test_masked_cfg2(gpu):
    """T 32768, D 128, 32/8 heads, structured K, 35% block list + block stats."""
    L, keep = W.cfg2()
    gq, gk, gv = to_gpu(L.q, L.k, L.v)
    for ns in (None, 1, 5):
        check_decode(L.q, L.k, L.v, L.scale, gq, gk, gv, keep=keep, num_splits=ns, label="cfg2 masked")
    plan = K.make_plan(keep.cuda())
    rms = K.decode(gq, gk, gv, L.scale, plan=plan, stats=True)
    rd = K.decode(gq, gk, gv, L.scale, stats=True)
    vis = keep.cuda().repeat_interleave(4, 1)
    assert torch.isinf(rms["blk_max"][~vis]).all() and (rms["blk_sum"][~vis] == 0).all(), \
        "masked stats touched a skipped block"
    assert torch.equal(rms["blk_max"][vis], rd["blk_max"][vis]) and torch.equal(rms["blk_sum"][vis], rd["blk_sum"][vis])
    M, S = O.block_stats(L.q, L.k, L.scale, keep=keep)
    x_dev = O.block_logw(rms["blk_max"].cpu().double(), rms["blk_sum"].cpu().double())
    x_ref = O.block_logw(M, S)
    fin = torch.isfinite(x_ref)
    assert torch.equal(torch.isfinite(x_dev), fin)
    assert (x_dev - x_ref)[fin].abs().max().item() <= LSE_TOL
    # per query head per block (max, LSE, mass) as the config asks
    mass_dev = torch.softmax(x_dev.masked_fill(~fin, -math.inf), -1)
    mass_ref = torch.softmax(x_ref, -1)
    assert (mass_dev - mass_ref).abs().max().item() <= 1e-4
    check_decode(L.q, L.k, L.v, L.scale, gq, gk, gv, label="cfg2 dense")


def _selection_margin(q, k, scale, rule, value):
    """How close the oracle's selection of this input comes to flipping: for top-p its cut's distance
    from the level (topp_heads), for tau the smallest |weight - tau|."""
    logw = O.block_logw(*O.block_stats(q, k, scale))
    if rule == "topp":
        return float(O.topp_heads(logw, value)[1].min())
    return float((torch.softmax(logw, -1) - value).abs().min())


def test_write_p_and_two_pass(gpu):
    """Pass 1's fp16 P, and the two-pass V-skip: the device selection identical to the oracle's
    select_blocks on the first seed whose oracle margin exceeds 1e-6 (a decision closer than that to its
    threshold can flip under float32 sums), the output exact attention over the selected blocks."""
    scale = 128 ** -0.5
    for rule, val in (("topp", 0.99), ("tau", 1e-4)):
        for seed in range(8, 40):
            q, k, v = rand_qkv(1, 32, 8, 3000, 128, seed=seed, sink_gap=True)
            margin = _selection_margin(q, k, scale, rule, val)
            if margin > 1e-6:
                break
        assert margin > 1e-6, f"every seed tried has a near tie ({margin:.2e})"
        gq, gk, gv = to_gpu(q, k, v)
        if rule == "topp":
            r = K.decode(gq, gk, gv, scale, stats=True, load_v=False, write_p=True)
            P = O.p_values(q, k, scale)
            err = (r["p"].cpu().double() - P).abs().max().item()
            assert err <= 1e-3, err                                  # fp16 P
        r2 = K.vskip_two_pass(gq, gk, gv, scale, rule=rule, value=val, out_f32=True)
        _, keep = O.vskip_two_pass(q, k, v, scale, rule=rule, value=val)
        keep_dev = r2["keep"].cpu()
        ref_out, _ = O.decode(q, k, v, scale, keep=keep_dev)
        e16 = O.rel_err(r2["out"].cpu(), ref_out)
        e32 = O.rel_err(r2["out_f32"].cpu(), ref_out)
        print(f"vskip2 {rule} seed {seed}: kept {keep.float().mean():.3f}, oracle margin {margin:.2e}, "
              f"bf16 {e16:.2e} f32 {e32:.2e}", flush=True)
        assert torch.equal(keep_dev, keep), (rule, int((keep_dev != keep).sum()))
        assert e16 <= BF16_TOL and e32 <= 5e-4          # fp16 P bounds the fp32 output error


@pytest.mark.parametrize("S", [1, 2, 3, 7, 64])
def test_pv_split_counts_and_list_edges(gpu, S):
    """Pass 2 directly against the oracle's pv (kernels/kvskip_kernel.cu:316-421) on random P,
    scales and lists: split counts giving each wavefront 0..many items (odd and even, the
    double-buffered loop's tail), out-of-range entries (skipped), an empty list, D 64 and 128."""
    g = torch.Generator().manual_seed(40 + S)
    for D, G in ((128, 4), (64, 8)):
        B, Hkv, T = 2, 3, 2900
        Hq, nb = Hkv * G, math.ceil(2900 / 64)
        v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
        P = torch.rand(B, Hq, nb * 64, generator=g).to(torch.float16)
        P[..., T:] = 0
        scale_b = torch.rand(B, Hkv, nb, G, generator=g)
        keep = torch.rand(B, Hkv, nb, generator=g) < 0.4
        keep[1, 2] = False                                       # an empty list
        bi = torch.zeros(B, Hkv, nb, dtype=torch.int32)
        bc = torch.zeros(B, Hkv, dtype=torch.int32)
        for b in range(B):
            for h in range(Hkv):
                idx = torch.nonzero(keep[b, h])[:, 0].to(torch.int32)
                if b == 0 and h == 1:                            # invalid entries are skipped
                    idx = torch.cat([idx, torch.tensor([nb, nb + 5, -1], dtype=torch.int32)])
                bi[b, h, :len(idx)] = idx[:nb]
                bc[b, h] = min(len(idx), nb)
        out, o32 = E.pv(P.cuda(), v.cuda(), scale_b.cuda().contiguous(), bi.cuda(), bc.cuda(), S, True)
        keep_eff = torch.zeros_like(keep)
        for b in range(B):
            for h in range(Hkv):
                ent = bi[b, h, :bc[b, h]].long()
                ent = ent[(ent >= 0) & (ent < nb)]
                keep_eff[b, h, ent] = True
        ref = O.pv(P, v, scale_b, keep_eff)
        assert O.rel_err(o32.cpu(), ref) <= 2e-5, (D, G, S)
        assert O.rel_err(out.cpu(), ref) <= BF16_TOL, (D, G, S)


def _same_kept_set(r, keep, z):
    """The blocks whose V single-pass V-skip read (v_keep) are the oracle rule's, except a block whose
    decision margin |z| (log units) is below float32 noise (1e-4); vcount is their count."""
    got = r["v_keep"].cpu()
    border = (z.abs() < 1e-4) & ~O.always_keep(keep.shape[-1], 2)
    assert not bool(((got != keep) & ~border).any()), int(((got != keep) & ~border).sum())
    assert torch.equal(r["v_tiles"].cpu().to(torch.int64), got.sum(-1).to(torch.int64))


@pytest.mark.parametrize("tau", [1e-4, 1e-3])
def test_vskip1_sink_and_lse_prev(gpu, tau):
    """bench/test_decode.py:131-151: kept set equals the fp64 rule's (except decisions within
    fp32 noise of the threshold), output vs fp64 over that set; with the sink bound and with an
    exact lse_prev."""
    q, k, v = rand_qkv(2, 32, 8, 2500, 128, seed=9, sink_gap=True)
    gq, gk, gv = to_gpu(q, k, v)
    scale = 128 ** -0.5
    lse_exact = torch.logsumexp(O.scores(q, k, scale), -1)
    for lp in (None, lse_exact.float()):
        r = K.vskip_one_pass(gq, gk, gv, scale, tau=tau, out_f32=True, count=True, keep=True,
                             lse_prev=None if lp is None else lp.cuda().contiguous())
        keep, z = O.vskip1_keep(q, k, scale, tau, 2, lse_prev=lp)
        _same_kept_set(r, keep, z)
        ref, lse = O.decode(q, k, v, scale, keep=r["v_keep"].cpu())
        e16 = O.rel_err(r["out"].cpu(), ref)
        e32 = O.rel_err(r["out_f32"].cpu(), ref)
        print(f"vskip1 tau {tau:g} lse_prev={lp is not None}: kept {keep.float().mean():.3f} "
              f"bf16 {e16:.2e} f32 {e32:.2e}", flush=True)
        assert e16 <= BF16_TOL and e32 <= F32_TOL
        assert (r["lse"].cpu().double() - lse).abs().max().item() <= LSE_TOL


def test_vskip1_cfg3(gpu):
    """T 65536, no sink, lse_prev = exact normaliser perturbed by +-5%, tau 1e-4."""
    L = W.cfg3()
    lse_exact = torch.logsumexp(O.scores(L.q, L.k, L.scale), -1)
    lp = W.perturbed_lse(lse_exact, seed=33)
    gq, gk, gv = to_gpu(L.q, L.k, L.v)
    r = K.vskip_one_pass(gq, gk, gv, L.scale, tau=1e-4, out_f32=True, count=True, keep=True, lse_prev=lp.cuda())
    keep, z = O.vskip1_keep(L.q, L.k, L.scale, 1e-4, 2, lse_prev=lp)
    _same_kept_set(r, keep, z)
    ref, _ = O.decode(L.q, L.k, L.v, L.scale, keep=r["v_keep"].cpu())
    e16, e32 = O.rel_err(r["out"].cpu(), ref), O.rel_err(r["out_f32"].cpu(), ref)
    print(f"cfg3 vskip1: V kept {keep.float().mean():.3f} bf16 {e16:.2e} f32 {e32:.2e}", flush=True)
    assert e16 <= BF16_TOL and e32 <= F32_TOL


def test_read_bw(gpu):
    x = torch.ones(1 << 24, dtype=torch.bfloat16, device="cuda")
    o = torch.zeros(1, dtype=torch.int32, device="cuda")
    K.ext().read_bw(x, o, 1024)
    torch.cuda.synchronize()
    assert int(o.item()) == 0


@pytest.mark.parametrize("engine", ["valu", "mfma"])
def test_qk_engines(gpu, engine, monkeypatch):
    """Both QK engines (v_dot2 VALU, MFMA) against the oracle: dense / masked + stats / stats-only /
    vskip1, D 64 and 128, G 4 and 7."""
    monkeypatch.setenv("KVSKIP_AMD_QK", engine)
    from kvskip_amd import ext as E
    for D, G in ((128, 4), (64, 4), (128, 7)):
        q, k, v = rand_qkv(1, 4 * G, 4, 1200, D, seed=100 + D + G, sink_gap=True)
        gq, gk, gv = to_gpu(q, k, v)
        scale = D ** -0.5
        check_decode(q, k, v, scale, gq, gk, gv, num_splits=6, label=f"{engine} D{D} G{G}")
        keep = W.random_block_list(1, 4, O.nblocks(1200), 0.5, seed=D + G)
        r = check_decode(q, k, v, scale, gq, gk, gv, keep=keep, num_splits=4, label=f"{engine} D{D} G{G} masked")
        rs = K.decode(gq, gk, gv, scale, plan=K.make_plan(keep.cuda()), stats=True, num_splits=4)
        M, S = O.block_stats(q, k, scale, keep=keep)
        x_dev = O.block_logw(rs["blk_max"].cpu().double(), rs["blk_sum"].cpu().double())
        fin = torch.isfinite(O.block_logw(M, S))
        assert torch.equal(torch.isfinite(x_dev), fin)
        assert (x_dev - O.block_logw(M, S))[fin].abs().max().item() <= LSE_TOL
        so = K.decode(gq, gk, gv, scale, stats=True, load_v=False, num_splits=3)
        assert torch.equal(torch.isfinite(so["blk_max"]).cpu(), torch.ones_like(fin))
        r1 = K.vskip_one_pass(gq, gk, gv, scale, tau=1e-3, out_f32=True, count=True, num_splits=5)
        keep1, z = O.vskip1_keep(q, k, scale, 1e-3, 2)
        ref1, _ = O.decode(q, k, v, scale, keep=keep1)
        assert O.rel_err(r1["out_f32"].cpu(), ref1) <= F32_TOL


def test_decode_op_phases(gpu):
    """DecodeOp: run() and splits() + merge() (the two launches of decode, exposed separately)
    give the same bits as ext.decode."""
    from kvskip_amd import ext as E
    L = W.cfg1(device="cuda")
    ref = E.decode(L.q, L.k, L.v, L.scale, None, None, False, True, 8, 2, False, False)
    op = E.DecodeOp(L.q, L.k, L.v, L.scale, 8)
    op.run()
    assert torch.equal(op.out, ref[0]) and torch.equal(op.lse, ref[1])
    op.out.zero_()
    op.lse.zero_()
    op.splits()
    op.merge()
    assert torch.equal(op.out, ref[0]) and torch.equal(op.lse, ref[1])


@pytest.mark.parametrize("num_splits", [1, 3, 8, 32])
def test_masked_stats_gaps(gpu, num_splits):
    """Masked statistics into NaN-poisoned buffers: listed blocks carry the dense pass's statistics
    and every skipped block reads (-inf, 0) -- leading, inner and trailing gaps, a one-entry list
    and an empty list -- with no fill by the caller."""
    from kvskip_amd import ext as E
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, T, D = 2, 8, 4, 64 * 40 - 17, 64
    nb = math.ceil(T / 64)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).cuda()
    lists = [[5, 6, 17, 30], [0], [], [nb - 1], [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 20, 38], list(range(nb)),
             [3, nb - 3], [12, 13, 14, 15]]
    bi = torch.zeros(B, Hkv, nb, dtype=torch.int32)
    bc = torch.zeros(B, Hkv, dtype=torch.int32)
    keep = torch.zeros(B, Hkv, nb, dtype=torch.bool)
    for i, lst in enumerate(lists):
        b, h = divmod(i, Hkv)
        bi[b, h, :len(lst)] = torch.tensor(lst, dtype=torch.int32)
        bc[b, h] = len(lst)
        keep[b, h, lst] = True
    f32 = dict(dtype=torch.float32, device="cuda")
    bufs = dict(out=torch.empty(B, Hq, D, dtype=torch.bfloat16, device="cuda"), lse=torch.empty(B, Hq, **f32),
                blk_max=torch.full((B * Hq * nb,), math.nan, **f32), blk_sum=torch.full((B * Hq * nb,), math.nan, **f32),
                part_acc=torch.empty(B * Hq * num_splits * D, **f32), part_ml=torch.empty(B * Hq * num_splits * 2, **f32))
    E.decode_into(q, k, v, 0.125, bufs, bi.cuda(), bc.cuda(), stats=True, num_splits=num_splits)
    bmax = bufs["blk_max"].view(B, Hq, nb).cpu()
    bsum = bufs["blk_sum"].view(B, Hq, nb).cpu()
    dense = E.decode(q, k, v, 0.125, None, None, True, True, 4, 2, False, False)
    vis = keep.repeat_interleave(Hq // Hkv, 1)
    assert not torch.isnan(bmax).any() and not torch.isnan(bsum).any(), "a block was left unwritten"
    assert (bmax[~vis] == -math.inf).all() and (bsum[~vis] == 0).all()
    assert torch.equal(bmax[vis], dense[2].cpu()[vis]) and torch.equal(bsum[vis], dense[3].cpu()[vis])
