"""fa_attention_splitk_noalloc: split-K with the library's static per-GPU workspace.

Called through the C ABI (ctypes, _hip.splitk_noalloc) and compared with fa_attention_splitk
(caller workspace) on the same inputs: the same kernels run on the same partials, so output and
LSE are equal bit for bit.  Two calls in a row, the second smaller, so the second runs on an
array that still holds the first call's contents.  Requests beyond the array's size fail with
a workspace error before anything is launched."""
import pytest
import torch

import fused_attn
from fused_attn import _hip
from helpers import TOL, announce, max_err, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def _pair(q, k, v, causal, split_len, **kw):
    want, want_lse = _hip.splitk(q, k, v, causal=causal, split_len=split_len, return_lse=True, **kw)
    got, got_lse = _hip.splitk_noalloc(q, k, v, causal=causal, split_len=split_len, return_lse=True, **kw)
    torch.cuda.synchronize()
    return want, want_lse, got, got_lse


def test_noalloc_equals_workspace_entry_point_on_two_calls():
    announce("noalloc: large then small call")
    gen = torch.Generator(device="cuda").manual_seed(21)
    # first call: decode-shaped, 40 partitions of 128 keys
    q = randn(2, 8, 1, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(2, 2, 5000, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(2, 2, 5000, 128, dtype=torch.bfloat16, gen=gen)
    want, want_lse, got, got_lse = _pair(q, k, v, False, 128)
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)
    assert max_err(got, orc.attention(q.cpu(), k.cpu(), v.cpu())) <= TOL[torch.bfloat16]
    # second call: smaller, causal, another head dim and dtype; the array still holds call 1's partials
    q2 = randn(1, 4, 3, 64, dtype=torch.float16, gen=gen)
    k2 = randn(1, 1, 700, 64, dtype=torch.float16, gen=gen)
    v2 = randn(1, 1, 700, 64, dtype=torch.float16, gen=gen)
    want, want_lse, got, got_lse = _pair(q2, k2, v2, True, 64)
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)
    assert max_err(got, orc.attention(q2.cpu(), k2.cpu(), v2.cpu(), causal=True)) <= TOL[torch.float16]


def test_noalloc_fp8_cache():
    announce("noalloc: fp8")
    gen = torch.Generator(device="cuda").manual_seed(22)
    q = randn(2, 8, 2, 128, dtype=torch.bfloat16, gen=gen)
    k8, ks = fused_attn.quantize_kv_fp8(randn(2, 2, 3000, 128, gen=gen))
    v8, vs = fused_attn.quantize_kv_fp8(randn(2, 2, 3000, 128, gen=gen))
    want, want_lse, got, got_lse = _pair(q, k8, v8, True, 256, k_scale=ks, v_scale=vs)
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)


def test_noalloc_rejects_requests_beyond_its_array():
    announce("noalloc: too large")
    # B=32 Hq=32 n_q=1 D=128 in 128-key partitions of 32768 keys: 32*32*256*(512+8) B = 136 MB > 64 MiB
    q = torch.zeros(32, 32, 1, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(32, 8, 32768, 128, dtype=torch.bfloat16, device="cuda")
    need = _hip.workspace_bytes(32, 32, 1, 128, 256)
    assert need > _hip.SPLITK_NOALLOC_MAX_BYTES
    with pytest.raises(RuntimeError, match="no-allocation entry point holds at most"):
        _hip.splitk_noalloc(q, k, k, split_len=128)
    # the same cache in 4096-key partitions fits (8 partials per row)
    out = _hip.splitk_noalloc(q, k, k, split_len=4096)
    torch.cuda.synchronize()
    assert torch.equal(out, _hip.splitk(q, k, k, split_len=4096))


def test_noalloc_with_caller_out_and_lse_allocates_nothing():
    """With the output and the LSE passed in, the call allocates no device memory: neither torch's
    allocator nor the device's free bytes change across it (after one warm-up call, whose first
    launch may load the kernels' code objects).  The results still equal the workspace entry point's."""
    announce("noalloc: caller out and lse, no allocation")
    gen = torch.Generator(device="cuda").manual_seed(23)
    q = randn(2, 8, 1, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(2, 2, 3000, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(2, 2, 3000, 128, dtype=torch.bfloat16, gen=gen)
    want, want_lse = _hip.splitk(q, k, v, split_len=256, return_lse=True)
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    _hip.splitk_noalloc(q, k, v, split_len=256, out=out, lse=lse)
    out.zero_()
    lse.zero_()
    torch.cuda.synchronize()
    alloc0 = torch.cuda.memory_allocated()
    free0, _ = torch.cuda.mem_get_info()
    got, got_lse = _hip.splitk_noalloc(q, k, v, split_len=256, out=out, lse=lse)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert torch.cuda.memory_allocated() == alloc0
    assert free1 == free0
    assert got is out and got_lse is lse
    assert torch.equal(out, want) and torch.equal(lse, want_lse)
