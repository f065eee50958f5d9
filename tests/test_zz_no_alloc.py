"""GPU: ftm_moe_forward_noalloc -- the whole layer on the library's static
device scratch instead of a caller workspace -- against ftm_moe_forward with a
workspace, through the C ABI: outputs and routing bit for bit (the same
kernels), on two calls in a row, the second with fewer tokens, and the size
limit refused before any launch."""
import ctypes

import pytest
import torch

from ftmoe import _native as nat
from ftmoe import synthetic as S

pytestmark = pytest.mark.gpu


def _noalloc(layer, x, ids=None, w=None, logits=None):
    out = torch.empty_like(x)
    rc = nat.lib().ftm_moe_forward_noalloc(ctypes.byref(layer.c()), x.data_ptr(), int(x.shape[0]), out.data_ptr(),
                                           nat.ptr(ids), nat.ptr(w), nat.ptr(logits), nat.stream_of(x))
    nat.check(rc, "ftm_moe_forward_noalloc")
    return out


@pytest.mark.parametrize("name,T1,T2", [("c3_full", 16, 2), ("c3_full", 64, 9), ("c3_fp8", 40, 5),
                                        ("c2_gptq", 20, 7), ("c4_mxfp4", 24, 1)])
def test_noalloc_matches_forward_with_workspace(gpu, name, T1, T2):
    cfg = S.CONFIGS["c3_fp8"] if name == "c3_full" else S.SMALL[name]
    syn = S.generate(cfg, T=T1, seed=T1 + T2, device=gpu)
    layer = S.build_layer(syn)
    for T in (T1, T2):
        x = syn.x[:T].contiguous()
        print(f"noalloc {name} T={T}", flush=True)
        ref, ids_r, w_r, lg_r = layer.forward(x, return_routing=True)
        ids, w, lg = torch.empty_like(ids_r), torch.empty_like(w_r), torch.empty_like(lg_r)
        got = _noalloc(layer, x, ids, w, lg)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (name, T)
        assert torch.equal(ids, ids_r) and torch.equal(w, w_r) and torch.equal(lg, lg_r), (name, T)
        again = _noalloc(layer, x)  # routing outputs are optional
        torch.cuda.synchronize()
        assert torch.equal(again, ref), (name, T)


def test_noalloc_alternating_streams(gpu):
    """Calls on two streams in turn (each ordered after the last by an event):
    each clears the scratch's control region on its own stream first, so
    every call matches the workspace forward."""
    syn = S.generate(S.SMALL["c3_fp8"], T=12, seed=31, device=gpu)
    layer = S.build_layer(syn)
    ref = layer.forward(syn.x)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=gpu), torch.cuda.Stream(device=gpu)]
    prev = torch.cuda.current_stream(gpu)
    for i in range(4):
        s = streams[i % 2]
        s.wait_stream(prev)
        with torch.cuda.stream(s):
            got = _noalloc(layer, syn.x)
        prev = s
        torch.cuda.synchronize()
        assert torch.equal(got, ref), i


def test_noalloc_refuses_layers_beyond_its_scratch(gpu):
    """C3 at 512 tokens needs 41 MiB of workspace, more than the 16 MiB
    scratch: FTM_ERR_WORKSPACE before anything is launched."""
    syn = S.generate(S.CONFIGS["c3_fp8"], T=1, seed=2, device=gpu)
    layer = S.build_layer(syn)
    x = torch.zeros(512, syn.cfg.H, dtype=torch.bfloat16, device=gpu)
    assert layer.workspace_bytes(512) > nat.NOALLOC_SCRATCH_BYTES
    out = torch.empty_like(x)
    rc = nat.lib().ftm_moe_forward_noalloc(ctypes.byref(layer.c()), x.data_ptr(), 512, out.data_ptr(), None, None,
                                           None, nat.stream_of(x))
    assert rc == nat.ERR_WORKSPACE
