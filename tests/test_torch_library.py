"""The ops as torch custom operators (torch.ops.sdv.*): schemas, fake-tensor propagation and
tracing, without a GPU (no compute calls).  The GPU side (opcheck, torch.compile against the
eager op) is tests/test_gpu_torch_library.py."""
from __future__ import annotations

import re

import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from specdec_amd.kernels import ops  # noqa: F401  (registers torch.ops.sdv)


def _schema(name):
    return str(getattr(torch.ops.sdv, name).default._schema)


def test_schemas_declare_mutation():
    assert "!" not in _schema("paged_attention")
    for name in ("quant_append", "paged_attention_append"):
        s = _schema(name)
        for arg in ("k_pages", "v_pages", "v_scales"):
            assert re.search(r"Tensor\(a\d+!\) " + arg + r"\b", s), (name, s)


def _decode_inputs(device, layers=None):
    B, H, KV, S, D, nb, T = 2, 12, 2, 5, 128, 40, 300
    lead = (layers,) if layers else ()
    q = torch.empty(lead + (B, H, S, D), dtype=torch.bfloat16, device=device)
    kp = torch.empty(lead + (nb, KV, D // 8, 16, 8), dtype=torch.bfloat16, device=device)
    vp = torch.empty(lead + (nb, KV, D, 16), dtype=torch.uint8, device=device)
    vs = torch.empty(lead + (nb, KV, 16), dtype=torch.float32, device=device)
    bt = torch.empty((B, 20), dtype=torch.int32, device=device)
    sl = torch.empty((B,), dtype=torch.int32, device=device)
    return q, kp, vp, vs, bt, sl, T


def test_fake_tensors_propagate_shapes():
    with FakeTensorMode():
        q, kp, vp, vs, bt, sl, T = _decode_inputs("cuda")
        out = torch.ops.sdv.paged_attention(q, kp, vp, vs, bt, sl, T)
        assert out.shape == q.shape and out.dtype == torch.bfloat16 and out.device == q.device
        out = torch.ops.sdv.paged_attention(q, kp, vp, vs, bt, None, T, True)
        assert out.shape == q.shape
        k_new = torch.empty((10, 2, 128), dtype=torch.bfloat16, device="cuda")
        out = torch.ops.sdv.paged_attention_append(q, kp, vp, vs, bt, sl, T, k_new, k_new, None, "rcp")
        assert out.shape == q.shape
        slots = torch.empty((10,), dtype=torch.int32, device="cuda")
        assert torch.ops.sdv.quant_append(k_new, slots, kp, vp, vs, k_new, "rcp") is None


def test_traced_graph_keeps_the_ops():
    """make_fx with fake tensors records the custom ops as graph nodes (not opaque Python)."""
    def step(q, kp, vp, vs, bt, sl, k_new, slots):
        torch.ops.sdv.quant_append(k_new, slots, kp, vp, vs, k_new, "rcp")
        return torch.ops.sdv.paged_attention(q, kp, vp, vs, bt, sl, 300) * 2

    q, kp, vp, vs, bt, sl, _ = _decode_inputs("cpu")
    k_new = torch.zeros((10, 2, 128), dtype=torch.bfloat16)
    slots = torch.zeros((10,), dtype=torch.int32)
    gm = make_fx(step, tracing_mode="fake")(q, kp, vp, vs, bt, sl, k_new, slots)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert any("sdv.quant_append" in t for t in targets), targets
    assert any("sdv.paged_attention" in t for t in targets), targets
