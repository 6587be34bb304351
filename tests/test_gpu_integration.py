"""The ctypes stub of INTEGRATION.md, executed as written (library path filled in), gives the
same attention as the oracle: the documented binding is a working one."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ROOT, announce
from helpers import assert_close, build_pages, eager_ref, to_dev
from specdec_amd import _native
from specdec_amd import workloads as wl
from test_integration_doc import stub_source

pytestmark = pytest.mark.gpu


def test_integration_stub_runs(cuda_device):
    announce("INTEGRATION.md ctypes stub")
    src = stub_source().replace("<repo>/specdec-context-scaling_amd/specdec_amd/libsdv.so", str(_native.LIB_PATH))
    ns: dict = {}
    exec(compile(src, "INTEGRATION.md", "exec"), ns)
    g = wl.gen(131)
    kv, d, h, t = 2, 128, 12, 1000
    ks, vs = [wl.randn_bf16((kv, t, d), g)], [wl.randn_bf16((kv, t, d), g)]
    nb = -(-t // 16)
    rows = [list(torch.randperm(nb + 3, generator=g)[:nb].numpy())]
    kp, vp, sp = build_pages(ks, vs, nb + 3, rows)
    bt = np.array(rows, dtype=np.int32)
    q = wl.randn_bf16((1, h, 1, d), g)
    for _ in range(2):  # the cached workspace is reused: its sync prefix must be zero again
        out = ns["paged_attention"](q.to(cuda_device), to_dev(kp, cuda_device), to_dev(vp, cuda_device),
                                    to_dev(sp, cuda_device), to_dev(bt, cuda_device),
                                    to_dev(np.array([t], dtype=np.int32), cuda_device), t)
        torch.cuda.synchronize()
        assert_close(out.cpu(), eager_ref(q, ks[0][None], vs[0][None], d), "stub")
