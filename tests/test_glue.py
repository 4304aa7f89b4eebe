"""Decoder glue kernels against fp32 torch restatements, at the config-5
shapes (d = 3584, 28 query / 4 KV heads of 128, 576-position cache) and a
small one (head_dim 64), including a position at the end of the cache."""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("rows,n", [(1, 3584), (3, 256), (2, 9000)])
@pytest.mark.parametrize("with_delta", [True, False])
def test_add_rmsnorm(gpu, rows, n, with_delta):
    from metal_native import ops

    g = torch.Generator(device=gpu)
    g.manual_seed(n + rows)
    x = torch.randn((rows, n), device=gpu, generator=g).half()
    d = torch.randn((rows, n), device=gpu, generator=g).half() if with_delta else None
    w = (torch.randn(n, device=gpu, generator=g) * 0.1).half()
    x0 = x.clone()
    out = ops.add_rmsnorm(x, d, w, 1e-6)
    xs = (x0.float() + d.float()).half() if with_delta else x0
    assert torch.equal(x, xs)                                       # residual written back (fp16 add)
    xf = xs.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()).half()
    err = (out.float() - ref.float()).abs()
    assert float(err.max()) <= 2e-3 + 2e-3 * float(ref.float().abs().max())


def attention_ref(q, kc, vc, pos, scale):
    H, D = q.shape
    KVH = kc.shape[0]
    grp = H // KVH
    k = kc[:, : pos + 1].float()
    v = vc[:, : pos + 1].float()
    s = torch.matmul(q.view(KVH, grp, D).float(), k.transpose(1, 2)) * scale
    return torch.matmul(torch.softmax(s, dim=-1), v).reshape(1, H * D)


@pytest.mark.parametrize("H,KVH,D,L,pos", [(28, 4, 128, 576, 512), (28, 4, 128, 576, 575), (28, 4, 128, 576, 0),
                                           (4, 2, 64, 32, 17), (8, 8, 64, 200, 130), (6, 2, 96, 80, 70)])
def test_attention_decode(gpu, H, KVH, D, L, pos):
    from metal_native import ops

    g = torch.Generator(device=gpu)
    g.manual_seed(H * D + pos)
    q = torch.randn((H, D), device=gpu, generator=g).half()
    kc = torch.randn((KVH, L, D), device=gpu, generator=g).half()
    vc = torch.randn((KVH, L, D), device=gpu, generator=g).half()
    p = torch.tensor([pos], device=gpu)
    scale = 1.0 / math.sqrt(D)
    out = ops.attention_decode(q, kc, vc, p, scale)
    ref = attention_ref(q, kc, vc, pos, scale)
    err = (out.float() - ref).abs()
    assert float(err.max()) <= 3e-3 + 3e-3 * float(ref.abs().max()), float(err.max())


@pytest.mark.parametrize("H,KVH,D,L,pos", [(28, 4, 128, 576, 512), (4, 2, 64, 32, 31)])
def test_rope_kv(gpu, H, KVH, D, L, pos):
    from metal_native import ops
    from metal_native.decoder import DecoderConfig, apply_rope, rope_tables

    cfg = DecoderConfig(heads=H, kv_heads=KVH, head_dim=D, max_len=L)
    cos, sin = rope_tables(cfg, gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(pos)
    qkv = torch.randn((1, (H + 2 * KVH) * D), device=gpu, generator=g).half()
    kc = torch.zeros((KVH, L, D), device=gpu, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    q = ops.rope_kv(qkv, cos, sin, torch.tensor([pos], device=gpu), kc, vc, H, KVH, D)
    flat = qkv[0]
    rq = apply_rope(flat[: H * D].view(H, D), cos[pos], sin[pos])
    rk = apply_rope(flat[H * D:(H + KVH) * D].view(KVH, D), cos[pos], sin[pos])
    assert (q.float() - rq.float()).abs().max() <= 2e-3
    assert (kc[:, pos].float() - rk.float()).abs().max() <= 2e-3
    assert torch.equal(vc[:, pos], flat[(H + KVH) * D:].view(KVH, D))
    assert float(kc[:, :pos].abs().sum()) == 0 and float(vc[:, pos + 1:].abs().sum()) == 0


@pytest.mark.parametrize("H,KVH,D,L,pos", [(28, 4, 128, 576, 512), (28, 4, 128, 576, 575), (28, 4, 128, 576, 63),
                                           (4, 2, 64, 32, 17), (8, 8, 64, 200, 0)])
def test_fused_rope_attention_matches_separate_kernels(gpu, H, KVH, D, L, pos):
    """One launch (rotary + cache write + attention + combine) against the
    separate rope_kv and attention_decode kernels: same output up to the
    split-combine order, same cache contents, on three successive calls on
    one workspace (the per-head counters must be left at zero)."""
    from metal_native import ops
    from metal_native.decoder import DecoderConfig, rope_tables

    cfg = DecoderConfig(heads=H, kv_heads=KVH, head_dim=D, max_len=L)
    cos, sin = rope_tables(cfg, gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(pos + D)
    kc0 = torch.randn((KVH, L, D), device=gpu, generator=g).half()
    vc0 = torch.randn((KVH, L, D), device=gpu, generator=g).half()
    assert ops.attention_decode_rope_supported(H, D, L)
    scale = 1.0 / math.sqrt(D)
    for rep in range(3):
        qkv = torch.randn((1, (H + 2 * KVH) * D), device=gpu, generator=g).half()
        p = torch.tensor([pos], device=gpu)
        k1, v1 = kc0.clone(), vc0.clone()
        q = ops.rope_kv(qkv, cos, sin, p, k1, v1, H, KVH, D)
        want = ops.attention_decode(q, k1, v1, p, scale)
        k2, v2 = kc0.clone(), vc0.clone()
        got = ops.attention_decode_rope(qkv, cos, sin, p, k2, v2, H, KVH, D, scale)
        assert torch.equal(k1, k2) and torch.equal(v1, v2)
        err = (got.float() - want.float()).abs()
        assert float(err.max()) <= 1e-3 * (1 + float(want.float().abs().max())), (rep, float(err.max()))


@pytest.mark.parametrize("N,K,epi,qt", [(4608, 3584, "bias", "int4"), (2 * 18944, 3584, "swiglu", "int4"),
                                        (3584, 18944, None, "int4"), (1000, 256, None, "int4"),
                                        (640, 512, "swiglu", "int4"), (4608, 3584, "bias", "int8"),
                                        (1000, 256, None, "int8"), (640, 512, "swiglu", "int8")])
@pytest.mark.parametrize("with_delta", [True, False])
def test_rmsnorm_fused_into_gemv(gpu, N, K, epi, qt, with_delta):
    """One launch (residual add + RMSNorm in the GEMV's staging) against
    add_rmsnorm followed by dequant_matmul: the residual bit for bit, the
    product within the matmul tolerance."""
    import numpy as np

    import metal_native as mn
    from metal_native import ops
    from oracle import mq_oracle as O

    rng = np.random.default_rng(N + K)
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float16)).to(gpu)
    d = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float16)).to(gpu) if with_delta else None
    w = torch.from_numpy((rng.standard_normal(K) * 0.1 + 1).astype(np.float16)).to(gpu)
    if qt == "int4":
        _, wp, s, z = O.make_int4_problem(1, K, N, 128, seed=K)
        g = 128
    else:
        _, wp, s, z, g = O.make_int8_problem(1, K, N, seed=K, g=128)
        z = rng.uniform(-0.01, 0.01, s.shape).astype(np.float16)
    wp, s, z = (torch.from_numpy(t).to(gpu) for t in (wp, s, z))
    b = torch.from_numpy(rng.standard_normal(N).astype(np.float16)).to(gpu) if epi == "bias" else None
    qc = 0 if qt == "int4" else 1
    assert ops._L.mq_rmsnorm_dequant_matmul_supported(N, K, g, qc, ops._EPILOGUES[epi]) == 1
    r1 = torch.empty_like(x)
    y1 = ops.rmsnorm_dequant_matmul(x, d, w, 1e-6, r1, wp, s, z, g, qt, epilogue=epi, bias=b)
    assert mn.last_path() == "rows"
    r2 = x.clone()
    h = ops.add_rmsnorm(r2, d, w, 1e-6)
    y2 = mn.dequant_matmul(h, wp, s, z, g, qt, epilogue=epi, bias=b)
    assert torch.equal(r1, r2)
    err = (y1.float() - y2.float()).abs()
    assert float(err.max()) <= 2e-2 + 2e-3 * float(y2.float().abs().max()), float(err.max())


@pytest.mark.parametrize("V,case", [(152064, "random"), (152064, "tie"), (5001, "nan"), (1000, "neginf"),
                                    (2048, "tie_last")])
def test_argmax_embed(gpu, V, case):
    """One fused launch: token = torch.argmax(logits) (NaN wins, ties go to the
    lowest index), pos + 1, x = embed row token; twice in a row, so the
    arrival counter left by the first call is exercised."""
    from metal_native import ops

    g = torch.Generator(device=gpu)
    g.manual_seed(V)
    d = 136
    embed = torch.randn((V, d), device=gpu, generator=g).half()
    ws = ops.argmax_embed_workspace(V, gpu)
    tok = torch.zeros(1, dtype=torch.int64, device=gpu)
    pos = torch.tensor([41], dtype=torch.int64, device=gpu)
    x = torch.empty((1, d), dtype=torch.float16, device=gpu)
    for rep in range(2):
        logits = torch.randn(V, device=gpu, generator=g).half()
        if case == "tie":
            logits[[777, 99999, 150000]] = 60.0
        elif case == "tie_last":
            logits[[2046, 2047]] = 60.0
        elif case == "nan":
            logits[[4000, 17]] = float("nan")
        elif case == "neginf":
            logits.fill_(float("-inf"))
        want = int(torch.argmax(logits.float()).item())
        ops.argmax_embed(logits, embed, tok, pos, x, ws)
        torch.cuda.synchronize()
        assert int(tok.item()) == want
        assert int(pos.item()) == 42 + rep
        assert torch.equal(x[0], embed[want])


@pytest.mark.parametrize("D", [64, 128])
def test_positions_past_the_cache_touch_nothing(gpu, D):
    """A device position at or past the cache end (a caller bug) writes no
    cache row and reads only rows that exist: the caches are unchanged and
    the attention output is the finite softmax over the whole cache."""
    from metal_native import ops
    from metal_native.decoder import DecoderConfig, rope_tables

    H, KVH, L = 8, 2, 256
    cfg = DecoderConfig(heads=H, kv_heads=KVH, head_dim=D, max_len=L)
    cos, sin = rope_tables(cfg, gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(D)
    kc = torch.randn((KVH, L, D), device=gpu, generator=g).half()
    vc = torch.randn((KVH, L, D), device=gpu, generator=g).half()
    qkv = torch.randn((1, (H + 2 * KVH) * D), device=gpu, generator=g).half()
    scale = 1.0 / math.sqrt(D)
    for pos in (L, L + 100):
        p = torch.tensor([pos], device=gpu)
        k1, v1 = kc.clone(), vc.clone()
        q = ops.rope_kv(qkv, cos, sin, p, k1, v1, H, KVH, D)
        out = ops.attention_decode(q, k1, v1, p, scale)
        k2, v2 = kc.clone(), vc.clone()
        out2 = ops.attention_decode_rope(qkv, cos, sin, p, k2, v2, H, KVH, D, scale)
        torch.cuda.synchronize()
        assert torch.equal(k1, kc) and torch.equal(v1, vc)
        assert torch.equal(k2, kc) and torch.equal(v2, vc)
        assert torch.isfinite(out.float()).all() and torch.isfinite(out2.float()).all()
        want = attention_ref(q, kc, vc, L - 1, scale)
        assert float((out.float() - want.float()).abs().max()) <= 1e-2
