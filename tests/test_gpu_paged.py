"""Paged (block-table) K/V decode on the HIP split-K kernel.

Paged K/V is a roadmap item of the reference (README.md:224) with no reference code, so
its result is defined as split-K decode over each sequence's gathered keys.  Two checks:
the fp32 oracle on the gathered keys (bars of the 16-bit dtypes), and bit equality with
the dense split-K kernel on the same keys and partitions: paging changes where a tile is
read from, not what is computed."""
import pytest
import torch

import fused_attn
from helpers import TOL, announce, max_err, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def _dense_and_paged(b, hq, hkv, nq, n, d, page, dtype, lens=None, seed=0, extra=3):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = randn(b, hq, nq, d, dtype=dtype, gen=gen)
    k = randn(b, hkv, n, d, dtype=dtype, gen=gen)
    v = randn(b, hkv, n, d, dtype=dtype, gen=gen)
    cpu_gen = torch.Generator().manual_seed(seed)
    kc, vc, bt, sl = fused_attn.paged_from_dense(k, v, page, seqlens=lens, extra_pages=extra, generator=cpu_gen)
    return q, k, v, kc, vc, bt, sl


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("page", [16, 32, 48, 64, 256])
@pytest.mark.parametrize("nq,causal", [(1, False), (4, True), (20, True)])
def test_paged_matches_oracle(dtype, d, page, nq, causal):
    announce(f"paged oracle {dtype} d={d} page={page} nq={nq} causal={causal}")
    lens = [300, 0, 1000, 64]
    q, k, v, kc, vc, bt, sl = _dense_and_paged(4, 8, 2, nq, 1000, d, page, dtype, lens=lens)
    out = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=causal, max_seqlen_k=1000, split_len=128)
    torch.cuda.synchronize()
    ref = orc.attention_paged(q, kc, vc, bt, sl, causal=causal)
    assert out.shape == q.shape and not torch.isnan(out).any()
    assert max_err(out, ref) <= TOL[dtype]
    assert torch.all(out[1] == 0)  # zero-length sequence


@pytest.mark.parametrize("split_len", [64, 128, 512, None])
@pytest.mark.parametrize("nq,causal", [(1, False), (16, True), (20, True)])  # 1, 2 and 4 waves (64-key tiles)
def test_paged_is_bit_identical_to_dense_splitk(split_len, nq, causal):
    """Equal lengths: the paged kernel equals the dense split-K kernel bit for bit."""
    announce(f"paged == dense split_len={split_len} nq={nq} causal={causal}")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(3, 16, 4, nq, 777, 128, 64, torch.bfloat16)
    sk = split_len or fused_attn.ops.default_split_len(nq, 777, 3, 4, 4)
    dense = fused_attn.attention_splitk(q, k, v, causal=causal, split_len=sk)
    paged = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=causal, split_len=sk)
    assert torch.equal(dense, paged)


@pytest.mark.parametrize("page", [16, 48])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("split_len", [64, 128, 512, None])
@pytest.mark.parametrize("nq,causal", [(1, False), (16, True), (20, True)])
def test_paged_small_pages_bit_identical_to_dense_splitk(page, d, split_len, nq, causal):
    """Pages of 16 + 32k keys (vLLM's 16-key pages): the tile is fetched in 16-key page groups,
    and the result still equals the dense split-K kernel bit for bit."""
    announce(f"paged small pages == dense page={page} d={d} split_len={split_len} nq={nq} causal={causal}")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(2, 8, 2, nq, 700, d, page, torch.bfloat16)
    sk = split_len or fused_attn.ops.default_split_len(nq, 700, 2, 2, 4)
    dense = fused_attn.attention_splitk(q, k, v, causal=causal, split_len=sk)
    paged = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=causal, split_len=sk)
    assert torch.equal(dense, paged)


def test_paged_ragged_lengths_bit_identical_per_sequence():
    """Each sequence equals the dense split-K kernel run on that sequence alone (the extra
    empty partitions of shorter sequences weigh zero in the combine)."""
    announce("paged ragged per-sequence")
    lens = [1, 129, 640, 0, 1000, 64, 65]
    q, k, v, kc, vc, bt, sl = _dense_and_paged(len(lens), 8, 8, 1, 1000, 64, 128, torch.float16, lens=lens)
    paged = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=128)
    for b, n in enumerate(lens):
        if n == 0:
            assert torch.all(paged[b] == 0)
            continue
        dense = fused_attn.attention_splitk(q[b:b + 1], k[b:b + 1, :, :n].contiguous(), v[b:b + 1, :, :n].contiguous(),
                                            split_len=128)
        assert torch.equal(dense, paged[b:b + 1]), b


def test_paged_pool_layouts_and_views():
    """A [num_pages, page_size, Hkv, D] pool (passed as a transposed view) gives the same bits."""
    announce("paged pool layouts")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(2, 8, 2, 1, 500, 128, 64, torch.bfloat16)
    ref = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=128)
    kc_t = kc.transpose(1, 2).contiguous().transpose(1, 2)  # storage [P, page, Hkv, D]
    vc_t = vc.transpose(1, 2).contiguous().transpose(1, 2)
    assert not kc_t.is_contiguous()
    assert torch.equal(fused_attn.attention_paged(q, kc_t, vc_t, bt, sl, split_len=128), ref)
    wide = torch.zeros(bt.shape[0], bt.shape[1] + 5, dtype=torch.int32, device="cuda")
    wide[:, :bt.shape[1]] = bt  # a wider table (unused trailing columns)
    assert torch.equal(fused_attn.attention_paged(q, kc, vc, wide, sl, split_len=128), ref)


def test_paged_many_pages_per_partition():
    """32-key pages with long partitions: up to 255 block-table entries per workgroup (all four
    registers that hold them)."""
    announce("paged 32-key pages, long partitions")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(2, 4, 1, 1, 9000, 64, 32, torch.bfloat16)
    for split_len in (4096, 8128):
        dense = fused_attn.attention_splitk(q, k, v, split_len=split_len)
        paged = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=split_len)
        assert torch.equal(dense, paged), split_len
    with pytest.raises(RuntimeError, match="256 pages"):
        fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=8256)


def test_paged_16_key_pages_many_per_partition():
    """16-key pages: a 4032-key partition spans 254 of them (within the 256 block-table entries a
    workgroup holds), 4096 keys would need 258; without split_len the op caps the partition so
    that it fits."""
    announce("paged 16-key pages, long partitions")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(2, 4, 1, 1, 9000, 128, 16, torch.float16)
    dense = fused_attn.attention_splitk(q, k, v, split_len=4032)
    assert torch.equal(fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=4032), dense)
    with pytest.raises(RuntimeError, match="256 pages"):
        fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=4096)
    out = fused_attn.attention_paged(q, kc, vc, bt, sl)
    assert max_err(out, orc.attention_paged(q, kc, vc, bt, sl)) <= TOL[torch.float16]


def test_paged_out_of_pool_entries_read_as_zero_keys():
    announce("paged out-of-pool entries")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(2, 4, 2, 1, 256, 64, 64, torch.bfloat16)
    bad = bt.clone()
    bad[0, 1] = kc.shape[0] + 100
    bad[1, 3] = -5
    out = fused_attn.attention_paged(q, kc, vc, bad, sl, split_len=64)
    ref = orc.attention_paged(q, kc, vc, bad, sl)
    assert max_err(out, ref) <= TOL[torch.bfloat16]


def test_paged_empty_and_short_cases():
    announce("paged empty cases")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(2, 4, 2, 3, 100, 64, 32, torch.bfloat16, lens=[0, 0])
    assert torch.all(fused_attn.attention_paged(q, kc, vc, bt, sl) == 0)
    # more queries than keys, causal: rows before the first key are zero
    q, k, v, kc, vc, bt, sl = _dense_and_paged(1, 4, 2, 8, 5, 64, 32, torch.bfloat16)
    out = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=True)
    ref = orc.attention_paged(q, kc, vc, bt, sl, causal=True)
    assert max_err(out, ref) <= TOL[torch.bfloat16] and torch.all(out[:, :, :3] == 0)


def test_paged_decode_cache_size():
    """The decode workload (B=32, Hq=32, Hkv=8, 32768 keys, D=128) in 64-key pages: bit-identical
    to the dense split-K kernel at 128-key partitions and at the default policy."""
    announce("paged decode 32x32x32768x128")
    q, k, v, kc, vc, bt, sl = _dense_and_paged(32, 32, 8, 1, 32768, 128, 64, torch.bfloat16, extra=0)
    for split_len in (128, None):
        sk = split_len or fused_attn.ops.default_split_len(1, 32768, 32, 8, 4)
        dense = fused_attn.attention_splitk(q, k, v, split_len=sk)
        paged = fused_attn.attention_paged(q, kc, vc, bt, sl, max_seqlen_k=32768, split_len=sk)
        assert torch.equal(dense, paged), sk


def test_paged_lse_matches_dense_splitk_and_oracle():
    """The combine's LSE from a paged pool equals the dense split-K kernel's bit for bit (same partials) and
    the oracle's on the gathered keys; the zero-length sequence reports -inf."""
    announce("paged lse")
    lens = [300, 0, 1000, 64]
    q, k, v, kc, vc, bt, sl = _dense_and_paged(4, 8, 2, 4, 1000, 128, 64, torch.bfloat16, lens=lens)
    out, lse = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=True, max_seqlen_k=1000, split_len=128,
                                          return_lse=True)
    assert torch.all(torch.isneginf(lse[1]))
    for b, n in enumerate(lens):
        if n == 0:
            continue
        ks, vs = k[b:b + 1, :, :n].contiguous(), v[b:b + 1, :, :n].contiguous()
        dense, dlse = fused_attn.attention_splitk(q[b:b + 1], ks, vs, causal=True, split_len=128, return_lse=True)
        assert torch.equal(dense, out[b:b + 1]) and torch.equal(dlse, lse[b:b + 1]), b
        ref = orc.lse(q[b:b + 1].cpu(), ks.cpu(), causal=True).to(lse.device)
        assert (lse[b:b + 1] - ref).abs().max().item() < 2.0 ** -8
