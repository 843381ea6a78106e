"""q, k and v are checked against each other before anything reaches the C ABI or a GPU
(the reference's check_inputs, csrc/bindings.cpp:35-44, and _check, triton_fwd.py:217-222).
The kernels take head_dim and batch from q and the K/V dtype, lengths and heads from k, so a
mismatched V or K would otherwise be read past the end of its buffer.  CPU only: every case
raises before the GPU requirement, which the last tests show by reaching it."""
import pytest
import torch

from fused_attn import _hip

FP8 = getattr(torch, "float8_e4m3fn", None)


def t(*shape, dtype=torch.bfloat16):
    return torch.zeros(*shape, dtype=dtype)


DENSE_BAD = [
    # (q, k, v, message fragment)
    (t(2, 8, 16, 64), t(2, 2, 32, 64), t(2, 2, 32, 64, dtype=torch.float16), "same dtype"),
    (t(2, 8, 16, 64), t(2, 2, 32, 64), t(2, 2, 31, 64), "same shape"),
    (t(2, 8, 16, 64), t(2, 2, 32, 32), t(2, 2, 32, 32), "head_dim"),
    (t(4, 8, 16, 64), t(2, 2, 32, 64), t(2, 2, 32, 64), "batch"),
    (t(2, 8, 16, 64), t(2, 2, 32, 64)[0], t(2, 2, 32, 64)[0], "4-D"),
    (t(2, 8, 16, 64), t(2, 3, 32, 64), t(2, 3, 32, 64), "multiple"),
    (t(2, 8, 16, 64, dtype=torch.float16), t(2, 2, 32, 64), t(2, 2, 32, 64), "dtypes must match"),
]


@pytest.mark.parametrize("q,k,v,msg", DENSE_BAD)
def test_dense_mismatches_raise_before_launch(q, k, v, msg):
    with pytest.raises(RuntimeError, match=msg):
        _hip.fwd(q, k, v)


@pytest.mark.parametrize("q,k,v,msg", DENSE_BAD)
def test_splitk_mismatches_raise_before_launch(q, k, v, msg):
    with pytest.raises(RuntimeError, match=msg):
        _hip.splitk(q, k, v)


def test_varlen_mismatches_raise_before_launch():
    cu = torch.tensor([0, 16], dtype=torch.int32)
    q = t(16, 8, 64)
    for k, v, msg in [(t(16, 2, 64), t(15, 2, 64), "same shape"), (t(16, 2, 32), t(16, 2, 32), "head_dim"),
                      (t(16, 3, 64), t(16, 3, 64), "multiple"), (t(1, 16, 2, 64), t(1, 16, 2, 64), "3-D")]:
        with pytest.raises(RuntimeError, match=msg):
            _hip.varlen_fwd(q, k, v, cu, cu, 16, 16)


def test_paged_mismatches_raise_before_launch():
    q = t(2, 8, 1, 64)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    sl = torch.full((2,), 100, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="head_dim"):
        _hip.paged_decode(q, t(10, 2, 32, 128), t(10, 2, 32, 128), bt, sl, 100)
    with pytest.raises(RuntimeError, match="k_cache and v_cache"):
        _hip.paged_decode(q, t(10, 2, 32, 64), t(10, 2, 64, 64), bt, sl, 100)
    with pytest.raises(RuntimeError, match="dtypes must match"):
        _hip.paged_decode(q, t(10, 2, 32, 64, dtype=torch.float16), t(10, 2, 32, 64, dtype=torch.float16), bt, sl,
                          100)


def test_broadcast_kv_batch_passes_the_check():
    # a K/V batch of 1 is read with a zero batch stride for every query batch, as the
    # reference backend's matmul broadcasts it
    _hip._check_qkv(t(4, 8, 16, 64), t(1, 2, 32, 64), t(1, 2, 32, 64), "dense")


@pytest.mark.skipif(FP8 is None, reason="torch has no float8_e4m3fn")
def test_fp8_scale_shape_and_dtype_are_checked():
    q = t(2, 8, 1, 64)
    k8 = torch.zeros(2, 2, 200, 64, dtype=FP8)
    good = torch.ones(2, 2, 4)
    with pytest.raises(RuntimeError, match="k_scale must have shape"):
        _hip.splitk(q, k8, k8, k_scale=torch.ones(2, 2, 3), v_scale=good)
    with pytest.raises(RuntimeError, match="v_scale must have shape"):
        _hip.splitk(q, k8, k8, k_scale=good, v_scale=torch.ones(2, 4))
    with pytest.raises(RuntimeError, match="float tensor"):
        _hip.splitk(q, k8, k8, k_scale=good, v_scale=torch.ones(2, 2, 4, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="needs k_scale"):
        _hip.splitk(q, k8, k8)
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        _hip.splitk(q, k8, torch.zeros(2, 2, 200, 64, dtype=torch.bfloat16), k_scale=good, v_scale=good)


@pytest.mark.skipif(FP8 is None, reason="torch has no float8_e4m3fn")
def test_fp8_scales_of_any_float_dtype_become_fp32():
    k8 = torch.zeros(2, 2, 200, 64, dtype=FP8)
    ks = (torch.arange(16, dtype=torch.float32).reshape(2, 2, 4) + 0.5).to(torch.float16)
    vs = torch.arange(32, dtype=torch.float64).reshape(2, 2, 8)[..., ::2]  # strided fp64
    _hip._check_fp8_scales(k8, ks, vs)
    ks32, vs32 = _hip._prep_fp8_scales(k8, ks, vs)
    for got, src in ((ks32, ks), (vs32, vs)):
        assert got.dtype == torch.float32 and got.stride(-1) == 1
        assert torch.equal(got, src.to(torch.float32))
    assert ks32.stride() == vs32.stride()
    # fp32 scales with unit stride are passed through as they are
    f = torch.ones(2, 2, 4)
    a, b = _hip._prep_fp8_scales(k8, f, f.clone())
    assert a.data_ptr() == f.data_ptr()


@pytest.mark.skipif(FP8 is None, reason="torch has no float8_e4m3fn")
def test_paged_fp8_pools_and_scales_are_checked():
    q = t(2, 8, 1, 64)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    sl = torch.full((2,), 100, dtype=torch.int32)
    k8 = torch.zeros(10, 2, 64, 64, dtype=FP8)
    good = torch.ones(10, 2, 1)
    with pytest.raises(RuntimeError, match="need k_scale"):
        _hip.paged_decode(q, k8, k8, bt, sl, 100)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        k32 = torch.zeros(10, 2, 32, 64, dtype=FP8)
        _hip.paged_decode(q, k32, k32, bt, sl, 100, k_scale=torch.ones(10, 2, 1), v_scale=torch.ones(10, 2, 1))
    with pytest.raises(RuntimeError, match="k_scale must have shape"):
        _hip.paged_decode(q, k8, k8, bt, sl, 100, k_scale=torch.ones(2, 2, 2), v_scale=good)
    with pytest.raises(RuntimeError, match="v_scale must have shape"):
        _hip.paged_decode(q, k8, k8, bt, sl, 100, k_scale=good, v_scale=torch.ones(10, 1, 1))
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        _hip.paged_decode(q, k8, t(10, 2, 64, 64), bt, sl, 100, k_scale=good, v_scale=good)
    # consistent FP8 pools pass every check and stop at the device test
    with pytest.raises(RuntimeError, match="needs GPU tensors"):
        _hip.paged_decode(q, k8, k8, bt, sl, 100, k_scale=good, v_scale=good.half())


def test_valid_cpu_inputs_reach_the_gpu_requirement():
    # consistent shapes pass every check and stop at the device test, not earlier
    with pytest.raises(RuntimeError, match="needs GPU tensors"):
        _hip.fwd(t(2, 8, 16, 64), t(2, 2, 32, 64), t(2, 2, 32, 64))
    with pytest.raises(RuntimeError, match="needs GPU tensors"):
        _hip.splitk(t(2, 8, 1, 64), t(1, 2, 4096, 64), t(1, 2, 4096, 64))


OUT_BAD = [
    # (out, message fragment) for q = [2, 8, 1, 64] bf16
    (t(2, 8, 1, 32), "shape"),
    (t(2, 8, 2, 64), "shape"),
    (t(2, 8, 1, 64, dtype=torch.float16), "dtype"),
    (t(2, 8, 1, 128)[..., ::2], "unit D stride"),
    (t(2 * 8 * 64 + 1)[1:].view(2, 8, 1, 64), "8-byte"),
]


@pytest.mark.parametrize("out,msg", OUT_BAD)
def test_caller_outputs_are_checked_before_launch(out, msg):
    """A caller's ``out`` smaller than q, or of another dtype or layout, would be written past its end:
    the no-allocation path and the prefill entry points reject it before the C ABI."""
    q, k = t(2, 8, 1, 64), t(2, 2, 4096, 64)
    with pytest.raises(RuntimeError, match=msg):
        _hip.splitk_noalloc(q, k, k, out=out)
    with pytest.raises(RuntimeError, match=msg):
        _hip.fwd(q, k, k, out=out)


def test_caller_lse_is_checked_before_launch():
    q, k = t(2, 8, 1, 64), t(2, 2, 4096, 64)
    for lse, msg in [(torch.zeros(2, 8), "shape"), (torch.zeros(2, 8, 1, dtype=torch.float16), "float32"),
                     (torch.zeros(2, 8, 2)[..., :1].transpose(0, 1).contiguous().transpose(0, 1), None)]:
        if msg is None:  # a permuted but unit-stride LSE is accepted; the call then needs the GPU
            with pytest.raises(RuntimeError, match="GPU"):
                _hip.splitk_noalloc(q, k, k, lse=lse)
            continue
        with pytest.raises(RuntimeError, match=msg):
            _hip.splitk_noalloc(q, k, k, lse=lse)
