"""Split-K flash-decoding on the HIP kernels vs the fp32 oracle
(reference: tests/test_splitk_fp8.py:16-41), plus the 32k-key benchmark decode workloads."""
import pytest
import torch

import fused_attn
from fused_attn import _hip, ops
from helpers import FP8_TOL, TOL, announce, check_bars, max_err, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("num_splits", [1, 3, 8])
@pytest.mark.parametrize("b,h_q,h_kv,n_q,n_k,d",
                         [(1, 2, 1, 1, 1000, 64), (2, 4, 2, 4, 777, 64), (1, 2, 2, 16, 2048, 128),
                          (2, 32, 8, 1, 3000, 128), (1, 8, 1, 16, 2500, 128),
                          (2, 8, 2, 1, 1500, 256), (1, 4, 1, 16, 900, 256)])
def test_splitk_matches_oracle(b, h_q, h_kv, n_q, n_k, d, num_splits, causal, dtype):
    announce(f"splitk b={b} hq={h_q} hkv={h_kv} nq={n_q} nk={n_k} d={d} S={num_splits} causal={causal} {dtype}")
    torch.manual_seed(0)
    q = randn(b, h_q, n_q, d, dtype=dtype)
    k = randn(b, h_kv, n_k, d, dtype=dtype)
    v = randn(b, h_kv, n_k, d, dtype=dtype)
    out = fused_attn.attention_splitk_triton(q, k, v, causal=causal, num_splits=num_splits)
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal)
    assert out.dtype == q.dtype and out.shape == q.shape
    assert max_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("scale", [-0.3, 0.3])
@pytest.mark.parametrize("split_len", [64, 512])
def test_peaked_softmax_meets_the_reference_bar(scale, split_len):
    """Large |scale| makes each row follow a few V rows of magnitude ~4, where one bf16 ulp is 0.031:
    split-K (fp32 partials) and the prefill kernel stay within the reference's
    assert_close(atol=2e-2, rtol=2e-2) and within the plain max-abs bar of 2e-2.  Found by a random sweep
    (B=2 Hq=64 Hkv=8 nq=982 nk=790)."""
    announce(f"peaked softmax scale={scale} split={split_len}")
    gen = torch.Generator(device="cuda").manual_seed(1478)
    q = randn(2, 64, 982, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(2, 8, 790, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(2, 8, 790, 128, dtype=torch.bfloat16, gen=gen)
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), scale=scale)
    out = fused_attn.attention_splitk(q, k, v, scale=scale, split_len=split_len)
    check_bars(out, ref, TOL[torch.bfloat16])
    check_bars(fused_attn.attention(q, k, v, scale=scale), ref, TOL[torch.bfloat16])


@pytest.mark.parametrize("split_len", [64, 128, 192, 1024, 4096])
def test_split_len_sweep(split_len):
    announce(f"split_len={split_len}")
    torch.manual_seed(1)
    q = randn(2, 16, 2, 128, dtype=torch.bfloat16)
    k = randn(2, 4, 2333, 128, dtype=torch.bfloat16)
    v = randn(2, 4, 2333, 128, dtype=torch.bfloat16)
    out = fused_attn.attention_splitk(q, k, v, causal=True, split_len=split_len)
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True)) <= TOL[torch.bfloat16]


def test_splitk_is_chosen_for_decode_shapes():
    announce("dispatch decode")
    torch.manual_seed(0)
    q = randn(1, 8, 1, 64, dtype=torch.float16)
    k = randn(1, 2, 4096, 64, dtype=torch.float16)
    assert ops._pick_backend(q, k) == "hip" and ops._hip_kernel_for(q, k) == "splitk"
    assert ops._hip_kernel_for(randn(1, 8, 512, 64, dtype=torch.float16), k) == "fwd"
    out = fused_attn.attention(q, k, k, causal=True)
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), k.cpu(), causal=True)) <= TOL[torch.float16]


def test_forced_splitk_backend_name(monkeypatch):
    """FUSED_ATTN_BACKEND=splitk (a reference backend name) forces the split-K kernel for any shape."""
    announce("forced splitk")
    torch.manual_seed(0)
    q = randn(1, 4, 70, 64, dtype=torch.bfloat16)
    k = randn(1, 2, 300, 64, dtype=torch.bfloat16)
    monkeypatch.setenv("FUSED_ATTN_BACKEND", "splitk")
    assert ops._hip_kernel_for(q, k) == "splitk"
    out = fused_attn.attention(q, k, k, causal=True)
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), k.cpu(), causal=True)) <= TOL[torch.bfloat16]


def test_workspace_too_small_is_an_error():
    q = randn(1, 4, 1, 64, dtype=torch.bfloat16)
    k = randn(1, 2, 512, 64, dtype=torch.bfloat16)
    ws = torch.empty(4, dtype=torch.float32, device="cuda")
    need = _hip.workspace_bytes(1, 4, 1, 64, 4)
    assert need == 1 * 4 * 1 * 4 * (64 * 4 + 8)  # fp32 partials + fp32 (max, sum) pairs
    out = _hip.splitk(q, k, k, split_len=128, workspace=ws)  # too small -> the wrapper allocates its own
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), k.cpu())) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("fp8", [False, True])
def test_two_partitions_per_workgroup_with_an_odd_count(fp8):
    """Fine grids of multi-wave row blocks (and FP8 caches) run two partitions per workgroup:
    257 partitions leave the last workgroup one, causal spec-decode rows span two waves."""
    announce(f"two partitions per workgroup fp8={fp8}")
    gen = torch.Generator(device="cuda").manual_seed(3)
    n_k = 128 * 257 - 50
    q = randn(8, 32, 16, 128, dtype=torch.bfloat16, gen=gen)
    if fp8:
        k8, ks = fused_attn.quantize_kv_fp8(randn(8, 8, n_k, 128, gen=gen))
        v8, vs = fused_attn.quantize_kv_fp8(randn(8, 8, n_k, 128, gen=gen))
        out = fused_attn.attention_fp8(q, k8, ks, v8, vs, causal=True, split_len=128)
        ref = torch.empty(q.shape, device="cuda")
        for bi in range(8):
            ref[bi:bi + 1] = orc.attention_fp8(q[bi:bi + 1], k8[bi:bi + 1], ks[bi:bi + 1], v8[bi:bi + 1],
                                               vs[bi:bi + 1], causal=True)
        assert max_err(out, ref) <= FP8_TOL
    else:
        k = randn(8, 8, n_k, 128, dtype=torch.bfloat16, gen=gen)
        v = randn(8, 8, n_k, 128, dtype=torch.bfloat16, gen=gen)
        out = fused_attn.attention_splitk(q, k, v, causal=True, split_len=128)
        assert max_err(out, orc.attention_chunked(q, k, v, causal=True)) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("n_q,causal", [(1, False), (16, True)])
def test_benchmark_decode_workloads(n_q, causal):
    """B=32, Hq=32, Hkv=8, n_k=32768, D=128 bf16 with 128-key partitions (and the n_q=16 spec-decode shape)."""
    announce(f"benchmark decode nq={n_q} causal={causal}")
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = randn(32, 32, n_q, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(32, 8, 32768, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(32, 8, 32768, 128, dtype=torch.bfloat16, gen=gen)
    out = fused_attn.attention_splitk(q, k, v, causal=causal, split_len=128)
    ref = orc.attention_chunked(q, k, v, causal=causal)
    err = max_err(out, ref)
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err <= TOL[torch.bfloat16]
    # the public op picks split-K for this shape, with the default partition length
    split = ops.default_split_len(n_q, 32768, 32, 8, 4)
    op_out = fused_attn.attention(q, k, v, causal=causal)
    assert torch.equal(op_out, fused_attn.attention_splitk(q, k, v, causal=causal, split_len=split))
    assert max_err(op_out, ref) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("split_len", [128, None])
def test_long_context_decode(split_len):
    """262144 keys: 2048 partitions per (batch, kv-head) at 128-key partitions, and the default policy."""
    announce(f"long-context decode split={split_len}")
    gen = torch.Generator(device="cuda").manual_seed(6)
    q = randn(2, 32, 1, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(2, 8, 262144, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(2, 8, 262144, 128, dtype=torch.bfloat16, gen=gen)
    out = fused_attn.attention_splitk(q, k, v, split_len=split_len)
    ref = orc.attention_chunked(q, k, v, heads_per_chunk=4)
    err = max_err(out, ref)
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err <= TOL[torch.bfloat16]


def test_peaked_softmax_precision_splitk_vs_prefill():
    """The seed-1478 peaked case (|scale| 0.3: each row follows a few V rows of magnitude ~4) through the
    prefill kernel and split-K at two partition sizes, each against the fp32 oracle.  Split-K partials are
    fp32 (the reference's format, triton_splitk.py:156-158), so split-K adds no 16-bit rounding to the
    prefill kernel's: both meet the absolute bf16 bar, and split-K's error stays within the prefill
    kernel's plus a bf16-output-rounding margin."""
    gen = torch.Generator(device="cuda").manual_seed(1478)
    q = randn(2, 64, 982, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(2, 8, 790, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(2, 8, 790, 128, dtype=torch.bfloat16, gen=gen)
    for scale in (0.3, -0.3):
        announce(f"peaked precision scale={scale}")
        ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), scale=scale)
        e_pre = max_err(fused_attn.attention(q, k, v, scale=scale), ref)
        e64 = max_err(fused_attn.attention_splitk(q, k, v, scale=scale, split_len=64), ref)
        e512 = max_err(fused_attn.attention_splitk(q, k, v, scale=scale, split_len=512), ref)
        print(f"scale={scale}: max_abs_err prefill {e_pre:.4e}, split-K 64 {e64:.4e}, split-K 512 {e512:.4e}",
              flush=True)
        assert e_pre <= TOL[torch.bfloat16]
        for e in (e64, e512):
            assert e <= TOL[torch.bfloat16]
            assert e <= e_pre + 2.0 ** -6  # within half a bf16 step at |o| ~ 4 of the prefill kernel's error


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,h_q,h_kv,n_q,n_k,d,split_len",
                         [(2, 8, 2, 1, 3000, 128, 128), (1, 4, 1, 16, 2500, 64, 256), (2, 8, 2, 16, 8, 128, 64),
                          (1, 4, 2, 4, 1300, 256, 512),
                          # 32 or more partitions: partition-major partials, with one-, two- and four-wave
                          # workgroups (rows = G * n_q of 1, 64 and 128)
                          (2, 8, 8, 1, 5000, 64, 64), (1, 8, 2, 16, 4100, 128, 128), (1, 16, 2, 16, 9000, 128, 128)])
def test_splitk_lse_matches_oracle(b, h_q, h_kv, n_q, n_k, d, split_len, causal):
    """The combine's natural-log LSE [B, Hq, Nq] (the reference's WRITE_LSE quantity, triton_fwd.py:169-172);
    n_k < n_q causal rows see no key and report -inf."""
    announce(f"splitk lse b={b} hq={h_q} nq={n_q} nk={n_k} d={d} split={split_len} causal={causal}")
    torch.manual_seed(3)
    q = randn(b, h_q, n_q, d, dtype=torch.bfloat16)
    k = randn(b, h_kv, n_k, d, dtype=torch.bfloat16)
    v = randn(b, h_kv, n_k, d, dtype=torch.bfloat16)
    out, lse = fused_attn.attention_splitk(q, k, v, causal=causal, split_len=split_len, return_lse=True)
    ref = orc.lse(q.cpu(), k.cpu(), causal=causal).to(lse.device)
    assert lse.shape == (b, h_q, n_q) and lse.dtype == torch.float32
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(lse))
    # l sums the bf16-rounded P that the MFMA consumes: bf16-level relative error in l
    assert (lse[fin] - ref[fin]).abs().max().item() < 2.0 ** -8
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal)) <= TOL[torch.bfloat16]
    # the LSE does not depend on the partitioning
    _, lse1 = fused_attn.attention_splitk(q, k, v, causal=causal, split_len=max(64, -(-n_k // 64) * 64),
                                          return_lse=True)
    assert (lse1[fin] - lse[fin]).abs().max().item() < 2.0 ** -8
