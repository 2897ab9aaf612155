"""sg_moe_layer_noalloc (the layer on the library's own per-GPU scratch
array, no workspace argument) against sg_moe_layer (caller workspace)
through the C ABI: two calls in a row, the second with fewer tokens, each
bit-exact on indices, weights and outputs; plus the size limit."""
import ctypes

import numpy as np
import pytest
import torch

import sager_amd
from sager_amd import ops
from sager_amd.synth import q4k_random_np

pytestmark = pytest.mark.gpu
H, F, E, K = 2048, 512, 64, 8


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@pytest.fixture(scope="module")
def setup():
    rng = np.random.default_rng(2024)
    mats = [[torch.from_numpy(q4k_random_np(rng, F * H // 256)).cuda() for _ in range(E + 1)]
            for _ in range(3)]
    tabs = [torch.tensor([m.data_ptr() for m in row[:E]], dtype=torch.int64, device="cuda")
            for row in mats]
    sh = [row[E] for row in mats]
    gw = torch.from_numpy(rng.normal(0, 0.03, H).astype(np.float32)).cuda()
    return rng, mats, tabs, sh, gw


def _run(lib, tabs, sh, gw, x, lg, res, noalloc):
    T = x.shape[0]
    out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
    idx = torch.full((T, K + 1), -7, dtype=torch.int32, device="cuda")
    w = torch.full((T, K + 1), float("nan"), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    common = [_p(tabs[0]), _p(tabs[1]), _p(tabs[2]), _p(sh[0]), _p(sh[1]), _p(sh[2]), _p(gw),
              _p(x), _p(lg), _p(res), _p(out), _p(idx), _p(w)]
    if noalloc:
        st = lib.sg_moe_layer_noalloc(*common, T, H, F, E, K, 1.0, s)
    else:
        n = lib.sg_moe_layer_workspace_bytes(T, H, F, E, K)
        ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        st = lib.sg_moe_layer(*common, _p(ws), n, T, H, F, E, K, 1.0, s)
    assert st == 0, lib.sg_last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()


def test_noalloc_matches_workspace_entry_point(setup):
    rng, mats, tabs, sh, gw = setup
    lib = sager_amd.load()
    for T in (16, 4, 1):  # each call smaller than the one before
        x = torch.from_numpy(rng.normal(0, 1, (T, H)).astype(np.float32)).cuda()
        lg = torch.from_numpy(rng.normal(0, 1.5, (T, E)).astype(np.float32)).cuda()
        res = torch.from_numpy(rng.normal(0, 1, (T, H)).astype(np.float32)).cuda()
        ref = _run(lib, tabs, sh, gw, x, lg, res, noalloc=False)
        got = _run(lib, tabs, sh, gw, x, lg, res, noalloc=True)
        np.testing.assert_array_equal(got[1][:, :K], ref[1][:, :K])
        np.testing.assert_array_equal(got[2].view(np.uint32), ref[2].view(np.uint32))
        np.testing.assert_array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
        assert np.isfinite(got[0]).all()


def test_noalloc_rejects_shapes_beyond_scratch(setup):
    _, _, tabs, sh, gw = setup
    lib = sager_amd.load()
    x = torch.zeros((16, H), dtype=torch.float32, device="cuda")
    out = torch.zeros((16, H), dtype=torch.float32, device="cuda")
    idx = torch.zeros((16, 33), dtype=torch.int32, device="cuda")
    w = torch.zeros((16, 33), dtype=torch.float32, device="cuda")
    st = lib.sg_moe_layer_noalloc(_p(tabs[0]), _p(tabs[1]), _p(tabs[2]), None, None, None, None,
                                  _p(x), None, None, _p(out), _p(idx), _p(w), 16, H, 8192, E,
                                  32, 1.0, None)
    assert st == 8 and b"scratch" in lib.sg_last_error()
