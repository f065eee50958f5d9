#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ from the reference's own
quantizer and dequantizer functions, for the behaviour no closed form or
known-answer test pins (argmin tie order and log2/ceil exponents of the MXFP4
quantizer, the e8m0 scale at its extremes, the fp32 -> e4m3 cast inside the
block-FP8 quantizer, the per-channel INT8 quantizer's scale and rounding,
torch.topk's order on tied router scores).

Run in a container that holds the reference tree (it is read from
--reference, default /root/reference; nothing from it is copied):

    python tests/golden/make_golden.py [--only int8]

The functions are loaded from their source files alone
(python/freetoken/kernel/triton/mxfp4_linear.py:46-111,
python/freetoken/kernel/triton/fp8_block_linear.py:94-125,
python/freetoken/kernel/triton/int8_linear.py:34-43), which import only
torch.  The output files hold inputs and outputs only (numpy .npz, no
pickled objects).
"""
from __future__ import annotations

import argparse
import importlib.util
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load(path: str, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def mxfp4_inputs() -> np.ndarray:
    """[10, 128] fp32 rows of four 32-element blocks with the edge cases."""
    rng = np.random.RandomState(20260)
    w = (rng.randn(10, 128) * 0.02).astype(np.float32)
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0], np.float32)
    # block 0 of row 0: amax 6 (scale 1), every LUT midpoint and its negative
    w[0, :16] = np.concatenate([mids, -mids])
    w[0, 16:32] = np.array([0.0, -0.0, 0.5, -0.5, 1.0, 3.0, 4.0, -6.0] * 2, np.float32)
    # exact powers of two for amax / 6 (ceil(log2) on an exact integer)
    for j, amax in enumerate([12.0, 3.0, 6.0 * 2.0 ** -10, 6.0 * 2.0 ** 20]):
        w[1, 32 * j:32 * (j + 1)] = np.linspace(-amax, amax, 32, dtype=np.float32)
    # just above / below a power of two
    w[2, :32] = np.float32(6.0000005)
    w[2, 32:64] = np.float32(5.9999995)
    w[2, 64:96] = 0.0  # all-zero block: amax clamped to 1e-12
    w[2, 96:128] = np.float32(1e-40)  # subnormal amax, also clamped
    # exponent clamps: huge and tiny magnitudes
    w[3, :32] = np.float32(3e38)
    w[3, 32:64] = np.float32(1e-30)
    # midpoints at a non-unit scale (amax 24 -> scale 4)
    w[4, :32] = np.concatenate([mids * 4, -mids * 4, mids[:8] * 4, -mids[:8] * 4])
    return w


def fp8_inputs() -> np.ndarray:
    """[130, 200] fp32 (ragged 128x128 blocks) with rounding-boundary values."""
    rng = np.random.RandomState(20261)
    w = (rng.randn(130, 200) * 0.02).astype(np.float32)
    # block (0, 0): amax 448 (scale 1), values halfway between e4m3 codes
    w[0, :8] = np.array([448.0, 1.0625, 1.1875, 0.0, -0.0, 17.0, 19.0, -23.0], np.float32)
    w[1, :4] = np.array([0.0009765625, 0.00146484375, 0.0029296875, -0.001953125], np.float32)
    w[2, :] = 0.0
    return w


def int8_inputs() -> np.ndarray:
    """[8, 64] fp32 rows for the per-channel INT8 quantizer: half-way ties of
    w / scale (round half to even), a zero row (amax clamped to 1e-12), a
    subnormal row, huge magnitudes and random rows."""
    rng = np.random.RandomState(20262)
    w = (rng.randn(8, 64) * 0.02).astype(np.float32)
    # amax 127 -> scale exactly 1: w / scale lands on every .5 tie
    w[0, :] = np.concatenate([np.arange(-15.5, 16.5, 1.0, dtype=np.float32), np.float32([127.0, -127.0]),
                              np.linspace(-126.5, 126.5, 30, dtype=np.float32)])
    # amax 254 -> scale 2: ties at odd integers of w
    w[1, :] = np.concatenate([np.arange(-31.0, 33.0, 2.0, dtype=np.float32)[:32], np.float32([254.0]),
                              (rng.randn(31) * 50).astype(np.float32)])
    w[2, :] = 0.0
    w[3, :] = np.float32(1e-40) * np.sign(rng.randn(64)).astype(np.float32)
    w[4, :] = (rng.randn(64) * 1e30).astype(np.float32)
    return w


def topk_inputs() -> np.ndarray:
    """[6, 16] router logits with exact ties across the top-k boundary."""
    g = np.zeros((6, 16), np.float32)
    g[0] = 1.0                       # all equal
    g[1, [3, 7, 11]] = 2.0           # three tied maxima
    g[2, [0, 5, 9, 15]] = 1.5        # a tie at the k-th place (k = 4 of them, k = 2 picks)
    g[3] = np.arange(16) % 4         # repeating pattern
    g[4, [2, 3]] = -1.0
    g[5] = -np.arange(16, dtype=np.float32) // 2  # pairs of equal values
    return g


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--only", choices=("mxfp4", "fp8", "topk", "int8"), default=None,
                    help="write one fixture file (the others are left as they are)")
    args = ap.parse_args()
    kdir = os.path.join(args.reference, "python", "freetoken", "kernel", "triton")
    want = (lambda name: args.only in (None, name))
    wrote = []

    if want("mxfp4"):
        mx = _load(os.path.join(kdir, "mxfp4_linear.py"), "ref_mxfp4_linear")
        w = mxfp4_inputs()
        blocks, scales = mx.quantize_mxfp4_blocks(torch.from_numpy(w))
        # e8m0 extremes through the reference dequant: every code at scale bytes 0, 1, 126, 127, 254, 255
        codes = np.arange(256, dtype=np.uint8).reshape(16, 16)      # byte b holds codes b & 15, b >> 4
        dq_scales = np.array([0, 1, 126, 127, 254, 255], np.uint8)
        dq_blocks = np.stack([codes.reshape(-1)[i * 16:(i + 1) * 16] for i in range(16)])  # [16, 16]
        dq_in_b = np.broadcast_to(dq_blocks[None], (len(dq_scales), 16, 16)).copy()
        dq_in_s = np.broadcast_to(dq_scales[:, None], (len(dq_scales), 16)).copy()
        dq = mx.dequantize_mxfp4_blocks(torch.from_numpy(dq_in_b), torch.from_numpy(dq_in_s), out_dtype=torch.float32)
        np.savez(os.path.join(HERE, "mxfp4_quant.npz"), w=w, blocks=blocks.numpy(), scales=scales.numpy(),
                 dq_blocks=dq_in_b, dq_scales=dq_in_s, dq_out=dq.numpy())
        wrote.append("mxfp4_quant.npz")

    if want("fp8"):
        f8 = _load(os.path.join(kdir, "fp8_block_linear.py"), "ref_fp8_block_linear")
        w8 = fp8_inputs()
        q, s = f8.quantize_block_fp8(torch.from_numpy(w8))
        np.savez(os.path.join(HERE, "fp8_quant.npz"), w=w8, q_bits=q.view(torch.uint8).numpy(), scale=s.numpy())
        wrote.append("fp8_quant.npz")

    if want("int8"):
        i8 = _load(os.path.join(kdir, "int8_linear.py"), "ref_int8_linear")
        wi = int8_inputs()
        q, s = i8.quantize_int8_channel(torch.from_numpy(wi))
        np.savez(os.path.join(HERE, "int8_quant.npz"), w=wi, q=q.numpy(), scale=s.numpy())
        wrote.append("int8_quant.npz")

    if want("topk"):
        g = topk_inputs()
        probs = torch.softmax(torch.from_numpy(g), dim=-1)
        tw, ti = torch.topk(probs, 4, dim=-1)
        np.savez(os.path.join(HERE, "topk_ties.npz"), logits=g, top_w=tw.numpy(),
                 top_idx=ti.numpy().astype(np.int64))
        wrote.append("topk_ties.npz")
    print("wrote", wrote)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
