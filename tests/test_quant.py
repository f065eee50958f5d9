"""Product quantizers (ftmoe.quant, torch) against the oracle's numpy
restatements of the reference quantizers -- bit-exact, on the CPU."""
import numpy as np
import torch

import ftm_oracle as O
from ftm_helpers import np_

from ftmoe import quant


def test_block_fp8_matches_oracle_incl_ragged():
    g = torch.Generator().manual_seed(0)
    for shape in [(256, 256), (200, 130), (3, 1024, 512)]:
        w = torch.randn(*shape, generator=g) * 0.3
        q, s = quant.quantize_block_fp8(w)
        flat = w.reshape(-1, shape[-2], shape[-1])
        qf, sf = q.reshape(-1, shape[-2], shape[-1]), s.reshape(-1, *s.shape[-2:])
        for i in range(flat.shape[0]):
            oq, os_ = O.quantize_block_fp8(flat[i].numpy())
            np.testing.assert_array_equal(np_(qf[i]), oq)
            np.testing.assert_array_equal(sf[i].numpy(), os_)


def test_mxfp4_matches_oracle():
    g = torch.Generator().manual_seed(1)
    w = torch.randn(2, 40, 320, generator=g) * 0.5
    w[0, 0, :32] = 0.0  # all-zero block
    w[0, 1, :32] = torch.tensor([0.25, -0.25, 0.75, 6.0] * 8)  # exact LUT midpoints / powers of two
    b, s = quant.quantize_mxfp4_blocks(w)
    ob, os_ = O.quantize_mxfp4_blocks(w.numpy())
    np.testing.assert_array_equal(b.numpy(), ob)
    np.testing.assert_array_equal(s.numpy(), os_)


def test_int8_channel_and_pack_match_oracle():
    g = torch.Generator().manual_seed(2)
    w = torch.randn(64, 256, generator=g)
    q, s = quant.quantize_int8_channel(w)
    oq, os_ = O.quantize_int8_channel(w.numpy())
    np.testing.assert_array_equal(q.numpy(), oq)
    np.testing.assert_array_equal(s.numpy(), os_)
    np.testing.assert_array_equal(quant.pack_int8_to_int32(q).numpy(), O.pack_int8(oq))
    # round trip through the oracle's dequant is the per-row scale times the code
    back = O.dequantize_int8_packed(O.pack_int8(oq), os_[:, None], 256)
    np.testing.assert_array_equal(back, oq.astype(np.float32) * os_[:, None])


def test_gptq_quantizer_round_trip_and_layout():
    """No reference GPTQ quantizer exists: pin the layout (dequant with the
    oracle gives back each weight to within half a quantisation step) and the
    symmetric convention (stored zero nibble 7, scale = 2*amax/15 in fp16)."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn(512, 96, generator=g) * 0.02  # [K, N]
    qw, qz, sc = quant.quantize_gptq_int4(w, group_size=128)
    assert qw.shape == (64, 96) and qz.shape == (4, 12) and sc.shape == (4, 96) and sc.dtype == torch.float16
    assert (qz.view(torch.int32).numpy().view(np.uint32) == 0x77777777).all()
    amax = w.reshape(4, 128, 96).abs().amax(1)
    np.testing.assert_array_equal(sc.numpy(), (2 * amax / 15).to(torch.float16).numpy())
    back = O.dequantize_gptq_int4(qw.numpy(), qz.numpy(), sc.numpy(), 128)
    step = np.repeat(sc.float().numpy(), 128, axis=0)
    # half a step, plus the fp16 rounding of the scale at the clamped extreme code
    assert np.all(np.abs(back - w.numpy()) <= 0.5 * step * (1 + 2 ** -6))
