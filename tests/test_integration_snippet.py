"""The registry branch that INTEGRATION.md asks a maintainer to paste into
the reference's registry.py (src/micro_vllm/attention/operators/
registry.py:24-50), run as written (CPU only, no compute calls).

The block is read from the document, wrapped in a function like the
reference's ``get_attention_operator_class`` and executed three ways:
* with the package import forced to fail: a ``RuntimeError`` naming the
  package (and no ``UnboundLocalError`` from the ``except`` clause);
* with the library load forced to fail: a ``RuntimeError`` naming the HIP
  library, chained to the ``NativeLibraryError``;
* with both present: the operator class.
"""

from __future__ import annotations

import re
import sys
import textwrap
from pathlib import Path

import pytest

from micro_vllm_amd import _native
from micro_vllm_amd.attention.operators.base import AttentionOperator

DOC = Path(__file__).resolve().parents[1] / "INTEGRATION.md"


def registry_function():
    if not DOC.exists():
        pytest.skip("INTEGRATION.md is not in this copy of the tree")
    text = DOC.read_text()
    section = text.split("## 2. Register the operator", 1)[1]
    block = re.search(r"```python\n(.*?)```", section, flags=re.S).group(1)
    body = textwrap.indent(textwrap.dedent(block), "    ")
    source = (
        "def get_attention_operator_class(name):\n"
        f"{body}"
        "    raise ValueError(f'unsupported attention operator {name!r}')\n"
    )
    namespace: dict = {}
    exec(compile(source, str(DOC), "exec"), namespace)
    return namespace["get_attention_operator_class"]


def test_snippet_returns_the_operator_when_everything_is_present():
    lookup = registry_function()
    cls = lookup("mi355x_paged")
    assert issubclass(cls, AttentionOperator)
    with pytest.raises(ValueError):
        lookup("no_such_operator")


def test_snippet_turns_a_missing_package_into_runtime_error(monkeypatch):
    lookup = registry_function()
    # A None entry makes `import micro_vllm_amd` raise ModuleNotFoundError.
    for name in list(sys.modules):
        if name == "micro_vllm_amd" or name.startswith("micro_vllm_amd."):
            monkeypatch.setitem(sys.modules, name, None)
    with pytest.raises(RuntimeError, match="micro_vllm_amd package") as info:
        lookup("mi355x_paged")
    assert isinstance(info.value.__cause__, ModuleNotFoundError)


def test_snippet_turns_a_missing_library_into_runtime_error(monkeypatch):
    lookup = registry_function()

    def missing():
        raise _native.NativeLibraryError("HIP library not found")

    monkeypatch.setattr(_native, "load", missing)
    with pytest.raises(RuntimeError, match="MI355X HIP library") as info:
        lookup("mi355x_paged")
    assert isinstance(info.value.__cause__, _native.NativeLibraryError)
