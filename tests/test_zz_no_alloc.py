"""The allocation-free metric fit (pmg_fit_scale_shift_static, the fit with its workspace in a static device array)
against the workspace entry point pmg_fit_scale_shift, both through the C ABI: (s, t) and info bit for bit, on
consecutive calls whose second input is smaller (the static array keeps the previous call's contents)."""
import ctypes as C

import numpy as np
import pytest
import torch

from promptmoge_amd import _lib

from conftest import announce

pytestmark = pytest.mark.gpu


def _inputs(B, N, seed, dev):
    rng = np.random.default_rng(seed)
    z = rng.uniform(0.5, 6, size=(B, N)).astype(np.float32)
    t = (1.3 * z + 0.05 + rng.normal(0, 0.01, size=(B, N))).astype(np.float32)
    t = np.where(rng.random((B, N)) < 0.05, t * 2.5, t).astype(np.float32)
    m = (rng.random((B, N)) < 0.7).astype(np.uint8)
    return tuple(torch.from_numpy(a).to(dev) for a in (z, t, m))


def _fit_static(z, t, m, iters):
    B, N = z.shape
    st = torch.full((B, 2), -1.0, dtype=torch.float32, device=z.device)
    info = torch.full((B, 5), -1, dtype=torch.int32, device=z.device)
    _lib.call("pmg_fit_scale_shift_static", z.data_ptr(), t.data_ptr(), m.data_ptr(), B, N, iters, 0.2, 32,
              st.data_ptr(), info.data_ptr(), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st.cpu().numpy(), info.cpu().numpy()


def _fit_workspace(z, t, m, iters):
    B, N = z.shape
    lib = _lib.lib()
    nbytes = lib.pmg_fit_workspace_bytes(N, iters)
    ws = torch.zeros((nbytes,), dtype=torch.uint8, device=z.device)
    st = torch.full((B, 2), -1.0, dtype=torch.float32, device=z.device)
    info = torch.full((B, 5), -1, dtype=torch.int32, device=z.device)
    _lib.call("pmg_fit_scale_shift", z.data_ptr(), t.data_ptr(), m.data_ptr(), B, N, iters, 0.2, 32, st.data_ptr(),
              info.data_ptr(), ws.data_ptr(), nbytes, C.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st.cpu().numpy(), info.cpu().numpy()


def test_static_fit_matches_workspace_fit_on_consecutive_calls(gpu):
    # (B, N, iters): the largest size the static array holds, then smaller inputs (fewer blocks, fewer rounds)
    for B, N, iters, seed in [(2, 1 << 19, 16, 1), (3, 60_000, 4, 2), (1, 307_200, 10, 3)]:
        announce(f"static fit B={B} N={N} iters={iters}")
        z, t, m = _inputs(B, N, seed, gpu)
        st_s, info_s = _fit_static(z, t, m, iters)
        st_w, info_w = _fit_workspace(z, t, m, iters)
        assert np.isfinite(st_s).all() and (info_s[:, 4] == 0).all()
        assert np.array_equal(st_s.view(np.uint32), st_w.view(np.uint32)), (st_s, st_w)
        assert np.array_equal(info_s, info_w)


def test_static_fit_refuses_sizes_beyond_its_scratch(gpu):
    z, t, m = _inputs(1, (1 << 19) + 1, 4, gpu)
    with pytest.raises(_lib.PmgError, match="static scratch"):
        _fit_static(z, t, m, 4)
    z, t, m = _inputs(1, 1000, 4, gpu)
    with pytest.raises(_lib.PmgError, match="static scratch"):
        _fit_static(z, t, m, 17)
