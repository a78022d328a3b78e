"""The no-allocation lm_head entry point (tt_matvec_argmax_noalloc) against the
workspace entry point (tt_matvec_argmax), called through the C ABI.

Two calls in a row on the same GPU, the second with a smaller matrix, so the second
call runs on the scratch array the first one left behind; logits, token index and
maximum value must equal the workspace entry point's bit for bit."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import f16_normal, rng, to_torch
from thintensor_amd import _lib

pytestmark = pytest.mark.gpu


def _run(lib, fn, w, x, logits, rows, cols, stream, partials=None):
    idx = torch.full((1,), -1, device=w.device, dtype=torch.int64)
    val = torch.full((1,), float("nan"), device=w.device, dtype=torch.float32)
    if partials is None:
        rc = fn(w.data_ptr(), _lib.F16, w.stride(0), x.data_ptr(), _lib.F16, logits.data_ptr(), _lib.F16, rows, cols,
                idx.data_ptr(), val.data_ptr(), stream)
    else:
        rc = fn(w.data_ptr(), _lib.F16, w.stride(0), x.data_ptr(), _lib.F16, logits.data_ptr(), _lib.F16, rows, cols,
                partials.data_ptr(), partials.numel(), idx.data_ptr(), val.data_ptr(), stream)
    _lib.check(rc, fn.__name__)
    return idx, val


def test_noalloc_argmax_matches_workspace_entry_point(device):
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    for rows, cols, seed in ((152064, 5120, 1), (4099, 2048, 2)):  # second call smaller
        print(f"noalloc argmax rows={rows} cols={cols}", flush=True)
        g = rng(seed)
        w = to_torch(f16_normal(g, (rows, cols), 0.02), device)
        x = to_torch(f16_normal(g, cols), device)
        need = int(lib.tt_matvec_argmax_partials(rows, cols))
        partials = torch.empty(need, device=device, dtype=torch.int64)
        logits_a = torch.empty(rows, device=device, dtype=torch.float16)
        logits_b = torch.empty(rows, device=device, dtype=torch.float16)
        ia, va = _run(lib, lib.tt_matvec_argmax, w, x, logits_a, rows, cols, stream, partials)
        ib, vb = _run(lib, lib.tt_matvec_argmax_noalloc, w, x, logits_b, rows, cols, stream)
        torch.cuda.synchronize(device)
        assert torch.equal(logits_a.view(torch.int16), logits_b.view(torch.int16))
        assert int(ia.item()) == int(ib.item()) == int(torch.argmax(logits_a.float()).item())
        assert torch.equal(va.view(torch.int32), vb.view(torch.int32))


def test_noalloc_argmax_rejects_bad_shape(device):
    lib = _lib.load()
    w = torch.zeros((8, 64), device=device, dtype=torch.float16)
    x = torch.zeros(64, device=device, dtype=torch.float16)
    idx = torch.zeros(1, device=device, dtype=torch.int64)
    rc = lib.tt_matvec_argmax_noalloc(w.data_ptr(), _lib.F16, 64, x.data_ptr(), _lib.F16, None, _lib.F16, 0, 64,
                                      idx.data_ptr(), None, None)
    assert rc != 0 and b"bad shape" in lib.tt_last_error()
