"""GPU: the reference's ``Moe(nn.Module)`` drop-in (python/freetoken/layers/moe.py:
29-83) end to end -- router logits from this library's router, the ``fused``
backend's LOWP routing and grouped experts -- against the oracle: the same
bf16 router logits (bit for bit), the routing from them and the experts,
output within |got - ref| <= 2e-2 + 1e-2 |ref|."""
import numpy as np
import pytest
import torch

import ftm_oracle as O
from ftm_helpers import ATOL, RTOL, assert_close, np_

from ftmoe.layers import Moe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,renorm,on_input", [(1, True, False), (7, True, False), (16, False, False),
                                               (40, True, True)])
def test_moe_module_matches_oracle(gpu, T, renorm, on_input):
    E, H, I, k = 32, 256, 128, 4
    torch.manual_seed(T)
    m = Moe(H, E, I, k, device=gpu, renormalize=renorm, apply_router_weight_on_input=on_input)
    with torch.no_grad():
        m.gate.weight.copy_((torch.randn(E, H) * 0.05).to(torch.bfloat16))
        m.w1.copy_((torch.randn(E, 2 * I, H) * 0.05).to(torch.bfloat16))
        m.w2.copy_((torch.randn(E, H, I) * 0.05).to(torch.bfloat16))
    x = torch.randn(2, T, H).to(torch.bfloat16).to(gpu)  # [..., H]: the output keeps the shape
    with torch.no_grad():
        out = m(x)
        logits = m.router_logits(x.reshape(-1, H))
    torch.cuda.synchronize()
    assert out.shape == x.shape and out.dtype == x.dtype
    xb = np_(x.reshape(-1, H).cpu())
    ref_logits = O.router_logits(xb, np_(m.gate.weight.detach().cpu()))
    np.testing.assert_array_equal(logits.float().cpu().numpy(), ref_logits)
    ids, w = O.route(ref_logits, k, "softmax_topk_lowp", renorm, weight_dt="bf16", prob_dt="bf16")
    p13 = O.OracleProj("bf16", np.ascontiguousarray(np_(m.w1.detach().cpu())), 2 * I, H)
    p2 = O.OracleProj("bf16", np.ascontiguousarray(np_(m.w2.detach().cpu())), H, I)
    ref = O.moe_experts(p13, p2, O.bf16_bits_to_f32(xb), ids, w, E=E, on_input=on_input)
    assert_close(out.reshape(-1, H).float().cpu().numpy(), ref, ATOL, RTOL, what="Moe module")
