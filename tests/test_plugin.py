"""CPU: the attention plugin's host side (kvskip_amd.attention, the reference's
src/kvskip_attn.py:68-147,481-520): configuration defaults, per-layer policies, the prefill route,
the growing cache's views, registration and the errors of the decode route. The decode modes run
the HIP kernels and are checked in tests/test_gpu_plugin.py."""

import math
from types import SimpleNamespace

import pytest
import torch

from kvskip_amd import attention as A
from kvskip_amd.planner import Policy, PostPlanner


def test_config_defaults_follow_the_reference():
    """src/kvskip_attn.py:116-140: the reference's defaults."""
    c = A.KvskipConfig()
    assert (c.mode, c.level, c.tau, c.delta, c.max_age, c.local) == ("dense", 0.99, 1e-4, 0.05, 32, 2)
    assert c.dense_layers == (0,) and c.dense_heads == () and c.index_heads == () and not c.index_union
    assert c.calib is None and c.calib_hold == 0 and c.calib_warm == () and not c.calib_free
    assert c.calib_kind == "logit" and c.calib_auto_ix is None and c.count and not c.record


def test_policy_per_layer():
    c = A.KvskipConfig(dense_heads=((1, 0), (2, 3)), index_heads=((1, 2),), index_union=True, calib=0.05,
                       calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.1)
    p1, p2, p3 = c.policy(1), c.policy(2), c.policy(3)
    assert p1.dense_heads == (0,) and p1.index_heads == (2,) and p1.flags(4) == [1, 0, 4, 0]
    assert p2.dense_heads == (3,) and p2.index_heads == () and p2.flags(4) == [0, 0, 0, 1]
    assert p3.flags(4) == [0, 0, 0, 0]
    assert p1.max_age_at(0) == 8 and p1.max_age_at(32) == 32 and p1.calib_kind == "peak" and p1.needs_index


def _attn_ref(q, k, v, scale, causal):
    """fp64 softmax attention with GQA, [B, H, S, D] in, [B, S, H, D] out."""
    B, Hq, S, D = q.shape
    G = Hq // k.shape[1]
    kk = k.double().repeat_interleave(G, 1)
    vv = v.double().repeat_interleave(G, 1)
    s = torch.einsum("bhsd,bhtd->bhst", q.double(), kk) * scale
    if causal:
        T = k.shape[2]
        i = torch.arange(S)[:, None] + (T - S)
        s = s.masked_fill(torch.arange(T)[None, :] > i, -math.inf)
    return torch.einsum("bhst,bhtd->bhsd", s.softmax(-1), vv).transpose(1, 2)


def test_prefill_goes_to_sdpa():
    """More than one query position: SDPA (causal), output [B, S, Hq, D]."""
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, S, D = 2, 8, 2, 5, 64
    q = torch.randn(B, Hq, S, D, generator=g)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    mod = SimpleNamespace(layer_idx=3, num_key_value_groups=Hq // Hkv, is_causal=True)
    out, w = A.kvskip_attention_forward(mod, q, k, v, None, scaling=0.125)
    assert out.shape == (B, S, Hq, D)
    torch.testing.assert_close(out.double(), _attn_ref(q, k, v, 0.125, True), rtol=1e-4, atol=1e-5)


def test_decode_route_errors():
    """A decode step never falls back to the CPU: host tensors are refused by the extension's checks;
    unknown modes raise; the refresh mode refuses policies it has no rule for."""
    q = torch.randn(1, 8, 1, 64).to(torch.bfloat16)
    k = torch.randn(1, 2, 128, 64).to(torch.bfloat16)
    mod = SimpleNamespace(layer_idx=1)
    saved = A.KVSKIP.mode
    try:
        A.KVSKIP.mode = "nonsense"
        with pytest.raises(ValueError):
            A.kvskip_attention_forward(mod, q, k, k, None, scaling=0.125)
        for mode in ("dense", "refresh", "refresh_fused"):
            A.KVSKIP.reset()
            A.KVSKIP.mode = mode
            with pytest.raises(Exception):
                A.kvskip_attention_forward(mod, q, k, k, None, scaling=0.125)
    finally:
        A.KVSKIP.mode = saved
        A.KVSKIP.reset()
    for bad in (dict(calib=0.1), dict(index_heads=(0,)), dict(calib_warm=(4, 2)), dict(calib_auto_ix=0.1)):
        with pytest.raises(ValueError):
            PostPlanner(Policy(**bad))


def test_register():
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface
    A.register()
    assert AttentionInterface._global_mapping["kvskip"] is A.kvskip_attention_forward
    assert "kvskip" in AttentionMaskInterface._global_mapping


def test_growing_cache_views():
    """Appends land in one buffer of whole 64-token blocks; the layer returns views of its first n
    tokens with head stride capacity * D; growth keeps the contents; crop shortens the views."""
    g = torch.Generator().manual_seed(3)
    cache = A.GrowingCache(capacity=200)
    B, H, D = 2, 3, 16
    ks, vs = [], []
    caps = []
    for t in (7, 1, 1, 300, 1, 400):
        k = torch.randn(B, H, t, D, generator=g)
        v = torch.randn(B, H, t, D, generator=g)
        ks.append(k)
        vs.append(v)
        kk, vv = cache.update(k, v, 0)
        n = sum(x.shape[2] for x in ks)
        assert kk.shape == (B, H, n, D) and cache.get_seq_length(0) == n
        torch.testing.assert_close(kk, torch.cat(ks, 2), rtol=0, atol=0)
        torch.testing.assert_close(vv, torch.cat(vs, 2), rtol=0, atol=0)
        cap = cache.layers[0]._kbuf.shape[2]
        assert cap % A.BLOCK == 0 and cap >= max(n, 200) and kk.stride(1) == cap * D and kk.stride(2) == D
        caps.append(cap)
    # first allocation: need 7 + 512 headroom -> 576 (whole blocks); the 400-token append (need 710)
    # grows to max(710 + 512, 2 * 576) -> 1280
    assert caps == [576] * 5 + [1280]
    cache.layers[0].crop(-5)
    assert cache.get_seq_length(0) == 705 and cache.layers[0].keys.shape[2] == 705
    cache.layers[0].crop(100)
    assert cache.get_seq_length(0) == 100
    torch.testing.assert_close(cache.layers[0].keys, torch.cat(ks, 2)[:, :, :100], rtol=0, atol=0)
