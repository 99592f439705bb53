"""GPU parity for the 8-bit-activation data formats around the path: the is_a_8bit repack
layout (reference gptq_marlin_repack.cu:225-335, awq_marlin_repack.cu:165-270) and the W4A8
code remap marlin_int4_fp8_preprocess (marlin_int4_fp8_preprocess.cu:8-97), bit for bit
against the oracle, through the torch ops and the C ABI."""
import numpy as np
import pytest
import torch

import oracle as O
from marlin_v100_amd import _custom_ops as ops
from marlin_v100_amd import capi

pytestmark = pytest.mark.gpu


def _codes(k, n, bits, seed):
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, 1 << bits, (k, n), generator=gen, dtype=torch.int32)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("k,n", [(32, 64), (256, 512), (1024, 4096), (96, 192)])
def test_gptq_repack_a8_layout(bits, k, n):
    print(f"case a8-gptq bits={bits} k={k} n={n}", flush=True)
    q = _codes(k, n, bits, k + n + bits)
    words = O.gptq_pack(q, bits).cuda()
    empty = torch.empty(0, dtype=torch.int32, device="cuda")
    got = ops.gptq_marlin_repack(words, empty, k, n, bits, True).cpu().numpy()
    assert got.shape == (k // 16, n * 16 * bits // 32)
    assert np.array_equal(got, O.a8_repack(q.numpy(), bits))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("k,n", [(64, 64), (256, 512), (96, 192)])
def test_awq_repack_a8_layout_equals_gptq(bits, k, n):
    print(f"case a8-awq bits={bits} k={k} n={n}", flush=True)
    q = _codes(k, n, bits, 3 * k + n)
    got = ops.awq_marlin_repack(O.awq_pack(q, bits).cuda(), k, n, bits, True).cpu().numpy()
    assert np.array_equal(got, O.a8_repack(q.numpy(), bits))
    # the C ABI entry, into a caller-provided buffer
    out = capi.awq_marlin_repack(O.awq_pack(q, bits).cuda(), k, n, bits, is_a_8bit=True)
    assert np.array_equal(out.cpu().numpy(), got)


def test_moe_repack_a8_layout_per_expert():
    e, k, n, bits = 3, 128, 256, 4
    qs = [_codes(k, n, bits, 100 + i) for i in range(e)]
    words = torch.stack([O.gptq_pack(q, bits) for q in qs]).cuda()
    perm = torch.empty((e, 0), dtype=torch.int32, device="cuda")
    got = ops.gptq_marlin_moe_repack(words, perm, k, n, bits, is_a_8bit=True).cpu().numpy()
    for i in range(e):
        assert np.array_equal(got[i], O.a8_repack(qs[i].numpy(), bits))


def test_a8_repack_rejects_act_order():
    k, n = 128, 64
    words = O.gptq_pack(_codes(k, n, 4, 1), 4).cuda()
    perm = torch.randperm(k).to(torch.int32).cuda()
    with pytest.raises(RuntimeError, match="Unsupported repack config"):
        ops.gptq_marlin_repack(words, perm, k, n, 4, True)


def test_int4_fp8_preprocess_reference_kat_in_place():
    """tests/test_marlin_dense.py:372-388 at the reference's size."""
    gen = torch.Generator().manual_seed(11)
    unpacked = torch.randint(0, 16, (2048, 2048), generator=gen, dtype=torch.int32)
    packed = (unpacked[:, ::2] * 16 + unpacked[:, 1::2]).to(torch.int8).view(torch.int32).cuda()
    res = ops.marlin_int4_fp8_preprocess(packed, None, True)
    want = torch.where(unpacked >= 8, unpacked - 8, 15 - unpacked)
    want = (want[:, ::2] * 16 + want[:, 1::2]).to(torch.int8).view(torch.int32)
    assert res.data_ptr() == packed.data_ptr()
    assert torch.equal(res.cpu(), want)


def test_int4_fp8_preprocess_out_of_place_keeps_input():
    gen = torch.Generator().manual_seed(12)
    q = torch.randint(-2**31, 2**31 - 1, (64, 96), generator=gen, dtype=torch.int32)
    qd = q.cuda()
    res = ops.marlin_int4_fp8_preprocess(qd, None, False)
    assert torch.equal(qd.cpu(), q)
    assert np.array_equal(res.cpu().numpy(), O.int4_fp8_preprocess(q.numpy()))


@pytest.mark.parametrize("k,nw,gs", [(128, 16, 32), (256, 64, 128), (64, 8, 8)])
def test_int4_fp8_preprocess_awq_zero_points(k, nw, gs):
    gen = torch.Generator().manual_seed(k + nw)
    q = torch.randint(-2**31, 2**31 - 1, (k, nw), generator=gen, dtype=torch.int32)
    z = torch.randint(-2**31, 2**31 - 1, (k // gs, nw), generator=gen, dtype=torch.int32)
    res = ops.marlin_int4_fp8_preprocess(q.cuda(), z.cuda(), False)
    assert np.array_equal(res.cpu().numpy(), O.int4_fp8_preprocess(q.numpy(), z.numpy()))
    out = capi.marlin_int4_fp8_preprocess(q.cuda(), z.cuda())
    assert torch.equal(out.cpu(), res.cpu())


def test_int4_fp8_preprocess_rejects_bad_group_size():
    q = torch.zeros((64, 8), dtype=torch.int32, device="cuda")
    z = torch.zeros((16, 8), dtype=torch.int32, device="cuda")  # group size 4
    with pytest.raises(RuntimeError, match="group_size % 8 != 0"):
        ops.marlin_int4_fp8_preprocess(q, z, False)
