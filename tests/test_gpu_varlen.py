"""Packed variable-length prefill on the HIP kernel vs the per-sequence fp32 oracle
(reference: tests/test_varlen.py:15-43), plus the 16-sequence benchmark workload and a
sentinel check that no row outside the sequences is written."""
import pytest
import torch

import fused_attn
from fused_attn import _hip
from helpers import TOL, announce, max_err, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lens", [[5, 33, 70], [1, 1, 1], [128], [64, 0, 17], [0], [0, 0, 3]])
@pytest.mark.parametrize("h_q,h_kv", [(4, 4), (8, 2)])
def test_varlen_matches_oracle(lens, causal, h_q, h_kv, dtype):
    announce(f"varlen lens={lens} causal={causal} hq={h_q} hkv={h_kv} {dtype}")
    torch.manual_seed(0)
    d = 64
    qs = [randn(n, h_q, d, dtype=dtype) for n in lens]
    ks = [randn(n, h_kv, d, dtype=dtype) for n in lens]
    vs = [randn(n, h_kv, d, dtype=dtype) for n in lens]
    q, cu_q, max_q = fused_attn.pack_varlen(qs)
    k, cu_k, max_k = fused_attn.pack_varlen(ks)
    v, _, _ = fused_attn.pack_varlen(vs)
    out = fused_attn.attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal)
    ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert max_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_cross_attention_lengths(dtype):
    """Different q and k lengths per sequence (chunked prefill against a KV cache)."""
    announce(f"varlen cross {dtype}")
    torch.manual_seed(0)
    lq, lk = [8, 16, 0, 5], [40, 16, 7, 3]
    q, cu_q, max_q = fused_attn.pack_varlen([randn(n, 4, 128, dtype=dtype) for n in lq])
    k, cu_k, max_k = fused_attn.pack_varlen([randn(n, 2, 128, dtype=dtype) for n in lk])
    v, _, _ = fused_attn.pack_varlen([randn(n, 2, 128, dtype=dtype) for n in lk])
    for causal in (False, True):
        out = fused_attn.attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal)
        ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal)
        assert max_err(out, ref) <= TOL[dtype]


def test_varlen_writes_only_sequence_rows():
    """Rows past cu_seqlens_q[-1] (padding in a larger buffer) keep their sentinel bits."""
    announce("varlen sentinel")
    torch.manual_seed(0)
    lens = [3, 0, 130, 1, 64]
    total, pad = sum(lens), 37
    q = randn(total + pad, 8, 128, dtype=torch.bfloat16)
    k = randn(total + pad, 2, 128, dtype=torch.bfloat16)
    v = randn(total + pad, 2, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    sentinel = torch.full((total + pad, 8, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    out = _hip.varlen_fwd(q, k, v, cu, cu, max(lens), max(lens), causal=True, out=sentinel)
    torch.cuda.synchronize()
    assert not torch.isnan(out[:total]).any()
    assert torch.isnan(out[total:]).all()
    ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), causal=True)
    assert max_err(out[:total], ref[:total]) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("lens", [[3, 0, 130, 1, 64], [4096, 17, 300]])
def test_varlen_output_with_8_byte_alignment_only(lens):
    """An output view whose base and head stride are 8-byte but not 16-byte aligned takes the kernel's
    8-byte store path: same bits as a fresh output, and the columns around the view keep their sentinel."""
    announce(f"varlen 8-byte aligned output lens={lens}")
    torch.manual_seed(1)
    total = sum(lens)
    q = randn(total, 8, 128, dtype=torch.bfloat16)
    k = randn(total, 2, 128, dtype=torch.bfloat16)
    v = randn(total, 2, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    ref = _hip.varlen_fwd(q, k, v, cu, cu, max(lens), max(lens), causal=True)
    buf = torch.full((total, 8, 132), float("nan"), dtype=torch.bfloat16, device="cuda")
    out = buf[:, :, 4:132]
    assert out.data_ptr() % 16 == 8 and (out.stride(1) * 2) % 16 == 8
    _hip.varlen_fwd(q, k, v, cu, cu, max(lens), max(lens), causal=True, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.isnan(buf[:, :, :4]).all()


def test_benchmark_varlen_workload():
    """16 sequences, lengths ~U[0, 4096] by seed with one 0 and one 1; Hq=32, Hkv=8, D=128, bf16, causal."""
    announce("benchmark varlen")
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(0, 4097, (16,), generator=g).tolist()
    lens[0], lens[1] = 0, 1
    total = sum(lens)
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = randn(total, 32, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(total, 8, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(total, 8, 128, dtype=torch.bfloat16, gen=gen)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    out = fused_attn.attention_varlen(q, k, v, cu, cu, max(lens), max(lens), causal=True)
    ref = orc.attention_varlen(q, k, v, cu, cu, causal=True)
    err = max_err(out, ref)
    print(f"lens={lens} max_abs_err={err:.3e}", flush=True)
    assert err <= TOL[torch.bfloat16]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lens", [[5, 33, 70], [64, 0, 17], [1, 0, 130]])
def test_varlen_lse(lens, causal):
    """LSE [Hq, total_q] per packed token equals logsumexp of that sequence's scores; rows with no key are -inf."""
    import math

    announce(f"varlen lse lens={lens} causal={causal}")
    torch.manual_seed(0)
    h_q, h_kv, d = 8, 2, 128
    qs = [randn(n, h_q, d, dtype=torch.bfloat16) for n in lens]
    ks = [randn(n + 3, h_kv, d, dtype=torch.bfloat16) for n in lens]
    q, cu_q, max_q = fused_attn.pack_varlen(qs)
    k, cu_k, max_k = fused_attn.pack_varlen(ks)
    out, lse = _hip.varlen_fwd(q, k, k, cu_q, cu_k, max_q, max_k, causal=causal, return_lse=True)
    assert lse.shape == (h_q, q.shape[0]) and lse.dtype == torch.float32
    assert torch.equal(out, fused_attn.attention_varlen(q, k, k, cu_q, cu_k, max_q, max_k, causal=causal))
    got = lse.cpu()
    cq, ck = cu_q.tolist(), cu_k.tolist()
    for i in range(len(lens)):
        nq, nk = cq[i + 1] - cq[i], ck[i + 1] - ck[i]
        if nq == 0:
            continue
        qf = q[cq[i]:cq[i + 1]].float().cpu().transpose(0, 1)
        kf = orc.expand_kv(k[ck[i]:ck[i + 1]].float().cpu().transpose(0, 1)[None], h_q // h_kv)[0]
        s = torch.matmul(qf, kf.transpose(-1, -2)) / math.sqrt(d)
        if causal:
            s = s.masked_fill(~orc.causal_mask(nq, nk), float("-inf"))
        ref = torch.logsumexp(s, dim=-1)
        g = got[:, cq[i]:cq[i + 1]]
        fin = torch.isfinite(ref)
        assert torch.equal(fin, torch.isfinite(g))
        # l sums the bf16-rounded P the MFMA consumes: bf16-level relative error in l
        assert (g[fin] - ref[fin]).abs().max().item() < 2.0 ** -8


@pytest.mark.parametrize("nseq,h_kv", [(1, 1), (3, 2), (4, 2), (5, 2), (9, 1), (4, 4), (17, 1)])
def test_varlen_group_counts_around_the_xcd_multiple(nseq, h_kv):
    """The varlen grid walks (sequence, kv-head) groups per XCD and is padded to a multiple of 8 groups:
    group counts below, at and above multiples of 8 (1, 6, 8, 10, 9, 16, 17), ragged lengths with
    several 128-query blocks, output and LSE against the oracle."""
    import math
    import random

    announce(f"varlen groups nseq={nseq} hkv={h_kv}")
    rng = random.Random(nseq * 10 + h_kv)
    lens = [rng.choice([0, 1, rng.randint(2, 400)]) for _ in range(nseq)]
    lens[0] = max(lens[0], 300)
    h_q, d = 4 * h_kv, 128
    torch.manual_seed(nseq)
    qs = [randn(n, h_q, d, dtype=torch.bfloat16) for n in lens]
    ks = [randn(n, h_kv, d, dtype=torch.bfloat16) for n in lens]
    vs = [randn(n, h_kv, d, dtype=torch.bfloat16) for n in lens]
    q, cu, mx = fused_attn.pack_varlen(qs)
    k, _, _ = fused_attn.pack_varlen(ks)
    v, _, _ = fused_attn.pack_varlen(vs)
    out, lse = _hip.varlen_fwd(q, k, v, cu, cu, mx, mx, causal=True, return_lse=True)
    ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), causal=True)
    assert max_err(out, ref) <= TOL[torch.bfloat16]
    c = cu.tolist()
    for i, n in enumerate(lens):
        if n == 0:
            continue
        qf = q[c[i]:c[i + 1]].float().cpu().transpose(0, 1)
        kf = orc.expand_kv(k[c[i]:c[i + 1]].float().cpu().transpose(0, 1)[None], 4)[0]
        sc = torch.matmul(qf, kf.transpose(-1, -2)) / math.sqrt(d)
        sc = sc.masked_fill(~orc.causal_mask(n, n), float("-inf"))
        assert (lse.cpu()[:, c[i]:c[i + 1]] - torch.logsumexp(sc, dim=-1)).abs().max().item() < 2.0 ** -8


def test_attention_triton_alias_gives_the_kernel_result():
    from fused_attn.triton_fwd import attention_triton, attention_varlen_triton

    announce("triton_fwd aliases")
    torch.manual_seed(0)
    q = randn(2, 8, 100, 128, dtype=torch.bfloat16)
    k = randn(2, 2, 100, 128, dtype=torch.bfloat16)
    o, lse = attention_triton(q, k, k, causal=True, return_lse=True)
    o2, lse2 = _hip.fwd(q, k, k, causal=True, return_lse=True)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    qs = [randn(n, 8, 128, dtype=torch.bfloat16) for n in (3, 50)]
    qp, cu, mx = fused_attn.pack_varlen(qs)
    kp, cuk, mk = fused_attn.pack_varlen([randn(n, 2, 128, dtype=torch.bfloat16) for n in (3, 50)])
    assert torch.equal(attention_varlen_triton(qp, kp, kp, cu, cuk, mx, mk, causal=True),
                       fused_attn.attention_varlen(qp, kp, kp, cu, cuk, mx, mk, causal=True))


def _bench_lengths():
    lens = torch.randint(0, 4097, (16,), generator=torch.Generator().manual_seed(0)).tolist()
    lens[0], lens[1] = 0, 1
    return lens


@pytest.mark.parametrize("case", ["bench16", "ragged", "cross"])
def test_varlen_rows_are_bit_identical_to_dense_calls(case):
    """cu_seqlens indexing is exact: every sequence's rows of attention_varlen, and of its LSE, equal a dense
    attention call on that sequence alone, bit for bit.  The varlen kernel runs 4-wave (128-row) blocks, as
    the dense kernel does below 4096 queries, so each row goes through the same tile sequence; only the
    workgroup schedule and the addressing differ.  Sequences of 0 and 1 tokens included."""
    announce(f"varlen bit-exact {case}")
    if case == "bench16":
        lq = lk = [n for n in _bench_lengths()]
        hq, hkv = 32, 8
    elif case == "ragged":
        lq = lk = [0, 1, 31, 32, 33, 127, 128, 129, 200, 1]
        hq, hkv = 8, 2
    else:  # chunked prefill against a cache: q shorter than k, causal alignment bottom-right
        lq, lk = [8, 1, 0, 100, 129], [40, 1, 7, 100, 300]
        hq, hkv = 8, 2
    if case == "bench16":  # dense calls stay below 4096 queries (the 4-wave dense kernel)
        lq = lk = [min(n, 4095) for n in lq]
    d = 128
    gen = torch.Generator(device="cuda").manual_seed(11)
    qs = [randn(n, hq, d, dtype=torch.bfloat16, gen=gen) for n in lq]
    ks = [randn(n, hkv, d, dtype=torch.bfloat16, gen=gen) for n in lk]
    vs = [randn(n, hkv, d, dtype=torch.bfloat16, gen=gen) for n in lk]
    q, cu_q, max_q = fused_attn.pack_varlen(qs)
    k, cu_k, max_k = fused_attn.pack_varlen(ks)
    v, _, _ = fused_attn.pack_varlen(vs)
    for causal in (True, False):
        out, lse = _hip.varlen_fwd(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal, return_lse=True)
        for i, (nq, nk) in enumerate(zip(lq, lk)):
            if nq == 0:
                continue
            qd = qs[i].transpose(0, 1)[None].contiguous()
            kd = ks[i].transpose(0, 1)[None].contiguous()
            vd = vs[i].transpose(0, 1)[None].contiguous()
            od, ld = _hip.fwd(qd, kd, vd, causal=causal, return_lse=True)
            s, e = int(cu_q[i]), int(cu_q[i + 1])
            assert torch.equal(out[s:e], od[0].transpose(0, 1)), (case, i, causal)
            assert torch.equal(lse[:, s:e], ld[0]), (case, i, causal)
