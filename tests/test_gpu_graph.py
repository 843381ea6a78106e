"""The HIP ops inside captured HIP graphs (torch.cuda.CUDAGraph), replayed several times.

A serving loop captures its decode step once and replays it.  The ops launch only
kernels on the current stream (no memsets, no host synchronisation), and their
workspaces come from torch's allocator, which serves a capture from the graph's own
pool.  Each replay runs after unrelated eager work and a synchronisation, and must
equal the eager result bit for bit."""
import pytest
import torch

import fused_attn
from helpers import announce, randn

pytestmark = pytest.mark.gpu


def _capture_and_replay(fn, inputs, eager, replays=3):
    """Capture fn() (reading the static `inputs`), replay `replays` times with fresh values
    copied into the inputs between replays; every replay must equal eager(fresh values)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):  # warm-up outside the graph (library load, allocator)
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    for r in range(replays):
        fresh = [torch.randn(t.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(100 + r))
                 .to(t.dtype) for t in inputs]
        for t, f in zip(inputs, fresh):
            t.copy_(f)
        junk = torch.randn(1 << 20, device="cuda").sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = eager()
        assert torch.isfinite(junk)
        assert torch.equal(out, want), f"replay {r} differs from eager"


def test_graph_splitk_decode():
    announce("graph split-K decode")
    q = randn(4, 32, 1, 128, dtype=torch.bfloat16)
    k = randn(4, 8, 4096, 128, dtype=torch.bfloat16)
    v = randn(4, 8, 4096, 128, dtype=torch.bfloat16)
    fn = lambda: fused_attn.attention_splitk(q, k, v, split_len=128)  # noqa: E731
    _capture_and_replay(fn, [q, k, v], fn)


def test_graph_decode_through_the_op():
    announce("graph attention op (decode-shaped, split-K)")
    q = randn(2, 16, 4, 64, dtype=torch.float16)
    k = randn(2, 4, 3000, 64, dtype=torch.float16)
    v = randn(2, 4, 3000, 64, dtype=torch.float16)
    fn = lambda: fused_attn.attention(q, k, v, causal=True)  # noqa: E731
    _capture_and_replay(fn, [q, k, v], fn)


def test_graph_prefill():
    announce("graph prefill")
    q = randn(1, 8, 700, 128, dtype=torch.bfloat16)
    k = randn(1, 2, 700, 128, dtype=torch.bfloat16)
    v = randn(1, 2, 700, 128, dtype=torch.bfloat16)
    fn = lambda: fused_attn.attention(q, k, v, causal=True)  # noqa: E731
    _capture_and_replay(fn, [q, k, v], fn)


def test_graph_varlen_prefill():
    announce("graph varlen prefill")
    lens = [300, 0, 1, 129, 77]  # 5 sequences x 2 kv-heads: the grid is padded to 16 groups
    gen = torch.Generator(device="cuda").manual_seed(1)
    q, cu, mx = fused_attn.pack_varlen([randn(n, 8, 128, dtype=torch.bfloat16, gen=gen) for n in lens])
    k, _, _ = fused_attn.pack_varlen([randn(n, 2, 128, dtype=torch.bfloat16, gen=gen) for n in lens])
    v, _, _ = fused_attn.pack_varlen([randn(n, 2, 128, dtype=torch.bfloat16, gen=gen) for n in lens])
    fn = lambda: fused_attn.attention_varlen(q, k, v, cu, cu, mx, mx, causal=True)  # noqa: E731
    _capture_and_replay(fn, [q, k, v], fn)


def test_graph_paged_decode():
    announce("graph paged decode")
    gen = torch.Generator(device="cuda").manual_seed(0)
    k = randn(3, 2, 1000, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(3, 2, 1000, 128, dtype=torch.bfloat16, gen=gen)
    kc, vc, bt, sl = fused_attn.paged_from_dense(k, v, 64, seqlens=[1000, 17, 600],
                                                 generator=torch.Generator().manual_seed(0))
    q = randn(3, 8, 1, 128, dtype=torch.bfloat16, gen=gen)
    # max_seqlen_k is passed: reading it from seqlens_k would synchronise inside the capture
    fn = lambda: fused_attn.attention_paged(q, kc, vc, bt, sl, max_seqlen_k=1000, split_len=128)  # noqa: E731
    _capture_and_replay(fn, [q, kc, vc], fn)


def test_graph_fp8_decode_and_quantiser():
    announce("graph fp8 quantise + decode")
    x = randn(2, 4, 2048, 128)
    q = randn(2, 16, 1, 128, dtype=torch.bfloat16)

    def fn():
        k8, ks = fused_attn.quantize_kv_fp8(x)
        return fused_attn.attention_fp8(q, k8, ks, k8, ks, split_len=256)

    _capture_and_replay(fn, [x, q], fn)
