"""The oracle and the product quantizers against golden vectors written by the
reference's own functions (tests/golden/make_golden.py, run in a container
that holds the reference; the .npz files hold inputs and outputs only).

They pin what neither a closed form nor the reference's known-answer tests
fix: the MXFP4 quantizer's argmin tie order and ceil(log2) exponents with
their clamps (python/freetoken/kernel/triton/mxfp4_linear.py:79-111), the
e8m0 scale at bytes 0, 1, 254 and 255 through the reference dequant
(:46-76, torch.exp2: 255 is inf, and 0 * inf is NaN), the fp32 -> e4m3 cast
of the block-FP8 quantizer (fp8_block_linear.py:94-125), and what
torch.topk (fused_moe.py:92-93) does on tied router scores."""
import os

import numpy as np
import torch

import ftm_oracle as O

from ftmoe import quant

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_mxfp4_quantizer_matches_reference_vectors():
    d = _load("mxfp4_quant.npz")
    ob, os_ = O.quantize_mxfp4_blocks(d["w"])
    np.testing.assert_array_equal(ob, d["blocks"])
    np.testing.assert_array_equal(os_, d["scales"])
    pb, ps = quant.quantize_mxfp4_blocks(torch.from_numpy(d["w"]))
    np.testing.assert_array_equal(pb.numpy(), d["blocks"])
    np.testing.assert_array_equal(ps.numpy(), d["scales"])
    # the vectors reach the zero-block clamp (amax 1e-12 -> byte 85) and the largest
    # finite fp32 exponent (3e38 -> byte 253)
    assert 85 in d["scales"] and 253 in d["scales"]


def test_mxfp4_dequant_at_e8m0_extremes_matches_reference_vectors():
    d = _load("mxfp4_quant.npz")
    with np.errstate(over="ignore", invalid="ignore"):
        out = O.dequantize_mxfp4_blocks(d["dq_blocks"], d["dq_scales"])
    np.testing.assert_array_equal(out, d["dq_out"])  # NaN positions must match too
    assert np.isinf(d["dq_out"][-1]).any() and np.isnan(d["dq_out"][-1]).any()


def test_block_fp8_quantizer_matches_reference_vectors():
    d = _load("fp8_quant.npz")
    oq, os_ = O.quantize_block_fp8(d["w"])
    np.testing.assert_array_equal(oq.view(np.uint8), d["q_bits"])
    np.testing.assert_array_equal(os_, d["scale"])
    pq, ps = quant.quantize_block_fp8(torch.from_numpy(d["w"]))
    np.testing.assert_array_equal(pq.view(torch.uint8).numpy(), d["q_bits"])
    np.testing.assert_array_equal(ps.numpy(), d["scale"])


def test_router_ties_select_the_same_scores_as_torch_topk():
    """torch.topk's order among tied scores is implementation-defined (on this
    CPU build an all-equal row selects experts 9-12, not 0-3); the oracle and
    the kernels break ties to the lower expert index.  What ties cannot change
    is the selected scores, so those are pinned; indices agree wherever no tie
    straddles the selection."""
    d = _load("topk_ties.npz")
    logits, k = d["logits"], d["top_idx"].shape[1]
    ids, w = O.route(logits, k, mode="softmax_topk", renormalize=False, weight_dt="f32")
    np.testing.assert_allclose(np.sort(w, axis=1), np.sort(d["top_w"], axis=1), rtol=1e-6, atol=0)
    for t in range(logits.shape[0]):
        kth = np.sort(logits[t])[::-1][k - 1]
        if np.sum(logits[t] == kth) == np.sum(logits[t][d["top_idx"][t]] == kth):
            # no tie across the boundary: the same experts
            assert set(ids[t].tolist()) == set(d["top_idx"][t].tolist()), t


def test_int8_quantizer_matches_reference_vectors():
    """Per-channel symmetric INT8 (int8_linear.py:34-43): scale = max(amax,
    1e-12) / 127, codes round half to even and clamp to +-127 -- on .5 ties,
    a zero row, a subnormal row and huge magnitudes."""
    d = _load("int8_quant.npz")
    q, s = O.quantize_int8_channel(d["w"])
    np.testing.assert_array_equal(q, d["q"])
    np.testing.assert_array_equal(s, d["scale"])
    pq, ps = quant.quantize_int8_channel(torch.from_numpy(d["w"]))
    np.testing.assert_array_equal(pq.numpy(), d["q"])
    np.testing.assert_array_equal(ps.numpy(), d["scale"])
    # the ties of row 0 (scale 1) round to even: -15.5 -> -16, -14.5 -> -14
    assert d["scale"][0] == 1.0 and d["q"][0, 0] == -16 and d["q"][0, 1] == -14
