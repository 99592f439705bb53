"""CPU checks of the layer-integration helpers (no GPU): the AWQ checkpoint conversion and
the kernel's can_implement rules (awq_marlin.py:75-130; marlin.py:35-64)."""
import torch

import oracle as O
from marlin_v100_amd.layers import (MarlinLinearKernel, MPLinearLayerConfig,
                                    convert_awq_to_standard_format)
from marlin_v100_amd.scalar_type import scalar_types


def test_convert_awq_to_standard_format_matches_gptq_packing():
    gen = torch.Generator().manual_seed(1)
    for bits in (4, 8):
        q = torch.randint(0, 1 << bits, (128, 64), generator=gen, dtype=torch.int32)
        z = torch.randint(0, 1 << bits, (2, 64), generator=gen, dtype=torch.int32)
        layer = torch.nn.Module()
        layer.qweight = torch.nn.Parameter(O.awq_pack(q, bits), requires_grad=False)
        layer.qzeros = torch.nn.Parameter(O.awq_pack(z, bits), requires_grad=False)
        convert_awq_to_standard_format(layer, "qweight", "qzeros", bits)
        assert torch.equal(layer.qweight.data, O.gptq_pack(q, bits))
        assert torch.equal(layer.qzeros.data, O.pack_cols(z, bits))


def test_can_implement_rules():
    ok = MPLinearLayerConfig((4096, 4096), (4096, 4096), scalar_types.uint4b8, torch.float16,
                             128, False, True)
    assert MarlinLinearKernel.can_implement(ok)[0]
    bad_type = MPLinearLayerConfig((4096, 4096), (4096, 4096), scalar_types.uint4b8,
                                   torch.float16, 128, True, False)
    assert not MarlinLinearKernel.can_implement(bad_type)[0]
    bad_n = MPLinearLayerConfig((4096, 96), (4096, 96), scalar_types.uint4b8, torch.float16,
                                128, False, False)
    assert "min_thread_n" in MarlinLinearKernel.can_implement(bad_n)[1]
    bad_act = MPLinearLayerConfig((4096, 4096), (4096, 4096), scalar_types.uint4b8,
                                  torch.float8_e4m3fn, 128, False, False)
    assert not MarlinLinearKernel.can_implement(bad_act)[0]
