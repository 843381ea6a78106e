"""torch.compile(fullgraph=True) over the custom ops on GPU tensors (reference:
tests/test_torch_compile.py:24-39, which compiles on CPU only).

Inductor checks a custom op's real output against the strides of its fake kernel
(``q.new_empty(q.shape)``, contiguous), so the HIP path must return that layout whatever the
input layout: contiguous inputs, the ``[B,N,H,D]`` storage viewed as ``[B,H,N,D]`` (one of the
prefill configurations), a decode-shaped call (the split-K kernel and its combine) and the
varlen op.  The compiled graph must give the eager result bit for bit."""
import pytest
import torch

import fused_attn
from helpers import announce, randn

pytestmark = pytest.mark.gpu


def _compiled(f):
    torch._dynamo.reset()
    return torch.compile(f, fullgraph=True)


def _dense_inputs(layout, dtype, gen):
    if layout == "contiguous":
        return (randn(2, 8, 256, 128, dtype=dtype, gen=gen), randn(2, 2, 256, 128, dtype=dtype, gen=gen),
                randn(2, 2, 256, 128, dtype=dtype, gen=gen))
    if layout == "bnhd_view":
        q = randn(2, 256, 8, 128, dtype=dtype, gen=gen).transpose(1, 2)
        k = randn(2, 256, 2, 128, dtype=dtype, gen=gen).transpose(1, 2)
        v = randn(2, 256, 2, 128, dtype=dtype, gen=gen).transpose(1, 2)
        assert not q.is_contiguous()
        return q, k, v
    # decode-shaped: 1 query against 4096 keys, the split-K path
    return (randn(4, 8, 1, 128, dtype=dtype, gen=gen), randn(4, 2, 4096, 128, dtype=dtype, gen=gen),
            randn(4, 2, 4096, 128, dtype=dtype, gen=gen))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["contiguous", "bnhd_view", "decode"])
def test_compiled_attention_equals_eager(layout, dtype):
    announce(f"compile attention {layout} {dtype}")
    gen = torch.Generator(device="cuda").manual_seed(31)
    q, k, v = _dense_inputs(layout, dtype, gen)

    def f(q, k, v):
        return fused_attn.attention(q, k, v, causal=True) * 2.0

    eager = f(q, k, v)
    got = _compiled(f)(q, k, v)
    torch.cuda.synchronize()
    assert got.shape == q.shape and got.dtype == dtype
    assert torch.equal(got, eager)


def test_compiled_attention_varlen_equals_eager():
    announce("compile attention_varlen")
    gen = torch.Generator(device="cuda").manual_seed(32)
    lens = [0, 1, 77, 300, 129]
    qs = [randn(n, 8, 128, dtype=torch.bfloat16, gen=gen) for n in lens]
    ks = [randn(n, 2, 128, dtype=torch.bfloat16, gen=gen) for n in lens]
    vs = [randn(n, 2, 128, dtype=torch.bfloat16, gen=gen) for n in lens]
    q, cu, mx = fused_attn.pack_varlen(qs)
    k, _, _ = fused_attn.pack_varlen(ks)
    v, _, _ = fused_attn.pack_varlen(vs)

    def g(q, k, v, cu):
        return fused_attn.attention_varlen(q, k, v, cu, cu, mx, mx, causal=True) * 2.0

    eager = g(q, k, v, cu)
    got = _compiled(g)(q, k, v, cu)
    torch.cuda.synchronize()
    assert got.shape == q.shape
    assert torch.equal(got, eager)
