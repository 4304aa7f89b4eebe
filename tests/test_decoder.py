"""Synthetic decoder on the quantized-linear kernels.

A tiny configuration is checked against an fp32 torch reference whose weights
are dequantized by the CPU oracle (one decode step: logits within the matmul
tolerance); HIP-graph replay must give the same tokens as eager steps.  The
full 28-layer configuration is tests/test_decoder_full.py.
"""

import numpy as np
import pytest
import torch

from oracle import mq_oracle as O

pytestmark = pytest.mark.gpu


def tiny():
    from metal_native.decoder import DecoderConfig

    return DecoderConfig(layers=2, d=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                         group_size=128, max_len=32)


def oracle_dequant(ql):
    K = ql.wp.shape[1] * 2
    w = O.dequant_int4(ql.wp.cpu().numpy(), ql.scales.cpu().numpy(), ql.zeros.cpu().numpy(), K, ql.g)
    return torch.from_numpy(w)


def test_decode_step_matches_oracle_reference(gpu):
    from metal_native.decoder import SyntheticDecoder

    m = SyntheticDecoder(tiny(), gpu, seed=3, prefilled=16)
    ref = m.reference_step(token=7, pos=16, dequant=oracle_dequant)
    tok = torch.tensor([7], device=gpu)
    pos = torch.tensor([16], device=gpu)
    nxt, logits = m.step(tok, pos, return_logits=True)
    torch.cuda.synchronize()
    got = logits[0].float()
    err = (got - ref).abs()
    bound = 1e-2 + 1e-3 * ref.abs()   # the matmul contract
    assert bool((err <= bound).all()), f"max err {err.max().item():.3g}"
    # greedy choice agrees wherever the reference's top-2 margin exceeds the tolerance
    top2 = torch.topk(ref, 2).values
    if (top2[0] - top2[1]).item() > 2e-2:
        assert int(nxt.item()) == int(torch.argmax(ref).item())


def test_graph_replay_matches_eager(gpu):
    from metal_native.decoder import SyntheticDecoder

    def run(graph: bool):
        m = SyntheticDecoder(tiny(), gpu, seed=5, prefilled=8)
        tok = torch.tensor([3], device=gpu)
        pos = torch.tensor([8], device=gpu)
        out = []
        if not graph:
            for _ in range(6):
                tok = m.step(tok, pos)
                pos = pos + 1
                out.append(int(tok.item()))
            return out
        s = torch.cuda.Stream(gpu)
        s.wait_stream(torch.cuda.current_stream(gpu))
        with torch.cuda.stream(s):
            m.step(tok, pos)  # warm-up (the step only writes cache slot `pos`, overwritten below)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            nxt = m.step(tok, pos)
            tok.copy_(nxt)
            pos.add_(1)
        pos.fill_(8)
        tok.fill_(3)
        for _ in range(6):
            g.replay()
            torch.cuda.synchronize()  # eager host work between replays
            out.append(int(tok.item()))
        return out

    assert run(False) == run(True)


def test_chained_graph_matches_eager(gpu):
    """The timed decode loop: step_chain (fused argmax + position + embedding
    row) captured once and replayed gives the eager steps' tokens."""
    from metal_native.decoder import SyntheticDecoder

    m = SyntheticDecoder(tiny(), gpu, seed=5, prefilled=8)
    tok = torch.tensor([3], device=gpu)
    pos = torch.tensor([8], device=gpu)
    want = []
    for _ in range(6):
        tok = m.step(tok, pos)
        pos = pos + 1
        want.append(int(tok.item()))
    m = SyntheticDecoder(tiny(), gpu, seed=5, prefilled=8)
    tok = torch.tensor([3], device=gpu)
    pos = torch.tensor([8], device=gpu)
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        m.start_chain(tok)
        m.step_chain(tok, pos)   # warm-up: writes cache slot 8, rewritten below
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        m.step_chain(tok, pos)
    tok.fill_(3)
    pos.fill_(8)
    m.start_chain(tok)
    got = []
    for _ in range(6):
        g.replay()
        torch.cuda.synchronize()  # eager host work between replays
        got.append(int(tok.item()))
    assert int(pos.item()) == 14
    assert got == want

