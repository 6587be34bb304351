"""The ctypes stub in INTEGRATION.md stays in step with include/sdv.h: it parses, and every
signature it declares has as many arguments as the header's declaration.  (The GPU test
tests/test_gpu_integration.py runs the stub itself.)"""
from __future__ import annotations

import ast
import re

from conftest import ROOT


def stub_source() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, re.S)
    stubs = [b for b in blocks if "ctypes.CDLL" in b]
    assert len(stubs) == 1, "expected one ctypes stub in INTEGRATION.md"
    return stubs[0]


def header_arity(name: str) -> int:
    h = (ROOT / "include" / "sdv.h").read_text()
    m = re.search(rf"\b{name}\((.*?)\);", h, re.S)
    assert m, name
    return len([a for a in m.group(1).split(",") if a.strip()])


def test_stub_parses_and_matches_header():
    src = stub_source()
    ast.parse(src)
    declared = dict(re.findall(r"_lib\.(sdv_\w+)\.argtypes = (.*)", src))
    assert {"sdv_paged_attention", "sdv_attention_workspace_size", "sdv_attention_workspace_init"} <= set(declared)
    for name, rhs in declared.items():
        rhs = rhs.strip()
        m = re.fullmatch(r"\[_I32\] \* (\d+)", rhs)
        if m:
            n = int(m.group(1))
        else:  # a list literal, possibly continued on the next line
            block = src[src.index(f"_lib.{name}.argtypes"):]
            lst = block[block.index("[") + 1:block.index("]")]
            n = len([x for x in lst.replace("\n", " ").split(",") if x.strip()])
        assert n == header_arity(name), (name, n, header_arity(name))
