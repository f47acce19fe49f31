"""The ``superl8`` interface (``superl8_serve_amd.shim``) exposes every name the
reference's paged-KV path and its tests look up on the external ``superl8``
package (tests/golden/superl8_names.json, listed from the reference's files by
tests/golden/make_superl8_names.py), accepts the call shapes those call sites
use, and refuses host tensors (there is no CPU implementation).  No GPU
needed: nothing here launches a kernel."""

from __future__ import annotations

import importlib
import inspect
import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from superl8_serve_amd import shim

NAMES = json.loads((Path(__file__).resolve().parent / "golden" / "superl8_names.json").read_text())["names"]

# Names outside the quantized paged-KV path, with the reason.
OUT_OF_SCOPE = {
    "superl8.QTensor": "quantized weight tensor of the model's linear layers (GEMM path, not the KV cache)",
}


def _resolve(dotted: str):
    parts = dotted.split(".")
    for cut in range(len(parts), 0, -1):
        try:
            obj = importlib.import_module(".".join(parts[:cut]))
        except ImportError:
            continue
        for attr in parts[cut:]:
            obj = getattr(obj, attr)
        return obj
    raise ImportError(dotted)


@pytest.fixture(scope="module", autouse=True)
def _installed():
    saved = {k: sys.modules.get(k) for k in shim._NAMES}
    shim.install()
    yield
    for k, v in saved.items():
        if v is None:
            sys.modules.pop(k, None)
        else:
            sys.modules[k] = v


def test_fixture_lists_the_cache_ops():
    for name in ("superl8.quantize_kv_write_paged", "superl8.attn_paged_decode_cached",
                 "superl8.attn_paged_decode_k8v3", "superl8.quant.rotation.rotate_last",
                 "superl8.quant.lloydmax.quantize_lloydmax"):
        assert name in NAMES


@pytest.mark.parametrize("name", sorted(NAMES))
def test_every_reference_name_resolves(name):
    if name in OUT_OF_SCOPE:
        pytest.skip(f"{name}: {OUT_OF_SCOPE[name]}")
    obj = _resolve(name)
    assert callable(obj), f"{name} is not callable"


def test_module_level_imports_of_the_cache_module_work():
    """kv_cache.py:35-36 and the call-time imports (502, 594, 613, 643)."""
    import superl8  # noqa: F401
    from superl8.quant.lloydmax import (dequantize_lloydmax, gaussian_codebook, pack_indices_lowbit,  # noqa: F401
                                        quantize_lloydmax, unpack_indices_lowbit)
    from superl8.quant.rotation import rotate_last  # noqa: F401

    assert shim.installed()
    assert callable(getattr(superl8, "attn_paged_decode_k8v3", None))  # the feature probe, kv_cache.py:700


def _binds(fn, *args, **kwargs):
    inspect.signature(fn).bind(*args, **kwargs)


def test_call_shapes_of_the_reference_call_sites():
    import superl8
    from superl8.quant import lloydmax, rotation

    x = object()
    _binds(superl8.quantize_kv_write_paged, x, x, x, x, x, x, x)                       # kv_cache.py:1073
    _binds(superl8.attn_paged_decode_cached, x, x, x, x, x, x, x, 16, max_context_len=1, scale=0.1)  # :1190
    _binds(superl8.attn_paged_decode_k8v3, x, x, x, x, x, x, x, x, 16, max_context_len=1, scale=0.1)  # :1170
    _binds(superl8.quantize_i8_rowwise, x)                                             # :601
    _binds(superl8.attn_int8_decode, x, x, x, scale=0.1)                               # :688
    _binds(superl8.attn_int8_fwd, x, x, x, causal=True, scale=0.1, window_left=-1)     # gqa_attention.py:122
    _binds(superl8.attn_int8_varlen, x, x, x, x, x, 4, 4, causal=True, scale=0.1)      # gqa_attention.py:91
    _binds(superl8.quantize_kv_cache, x, x)                                            # kv_cache.py:1231
    _binds(lloydmax.gaussian_codebook, 3, 128, "cuda")                                 # :504
    _binds(lloydmax.quantize_lloydmax, x, bits=3, block_size=128, dim=-1, codebook=x)  # :614-620
    _binds(lloydmax.pack_indices_lowbit, x, 3)                                         # :623
    _binds(lloydmax.unpack_indices_lowbit, x, 3, 128)                                  # :662
    _binds(lloydmax.dequantize_lloydmax, x, x, x, block_size=128, dim=-1)              # :663-669
    _binds(lloydmax.fake_quant_lloydmax, x, bits=3, block_size=128)                    # tests/test_k8v3_cache.py:108
    _binds(rotation.rotate_last, x)
    _binds(rotation.hadamard_matrix, 128, device="cpu", dtype=torch.float32)           # dist/pipeline.py:46


def test_hadamard_matrix_is_the_normalized_sylvester_matrix():
    from scipy.linalg import hadamard

    from superl8.quant.rotation import hadamard_matrix

    for d in (4, 32, 128):
        h = hadamard_matrix(d, device="cpu", dtype=torch.float64)
        assert np.array_equal(h.numpy(), hadamard(d) / np.sqrt(d))
    hadamard_matrix.cache_clear()  # dist/pipeline.py:65-70


def test_gaussian_codebook_matches_the_cache_codebook():
    from oracle import kv_oracle as O
    from superl8.quant.lloydmax import gaussian_codebook

    cb = gaussian_codebook(3, 128)
    assert cb.dtype == torch.float32 and cb.shape == (8,)
    assert np.array_equal(cb.numpy(), O.gaussian_codebook(3, 128))


@pytest.mark.parametrize("call", ["rotate_last", "quantize_i8_rowwise", "quantize_lloydmax", "pack_indices_lowbit",
                                  "quantize_kv_write_paged"])
def test_host_tensors_are_refused(call):
    import superl8
    from superl8.quant import lloydmax, rotation

    x = torch.zeros(2, 128, dtype=torch.float16)
    fns = {
        "rotate_last": lambda: rotation.rotate_last(x),
        "quantize_i8_rowwise": lambda: superl8.quantize_i8_rowwise(x),
        "quantize_lloydmax": lambda: lloydmax.quantize_lloydmax(x, bits=3, block_size=128, dim=-1),
        "pack_indices_lowbit": lambda: lloydmax.pack_indices_lowbit(torch.zeros(2, 128, dtype=torch.uint8), 3),
        "quantize_kv_write_paged": lambda: superl8.quantize_kv_write_paged(
            x[:, None], x[:, None], torch.zeros(1, 1, 16, 128, dtype=torch.int8), torch.ones(1, 1, 16),
            torch.zeros(1, 1, 16, 128, dtype=torch.int8), torch.ones(1, 1, 16), torch.zeros(2, dtype=torch.int32)),
    }
    with pytest.raises(RuntimeError, match="GPU tensor"):
        fns[call]()


def test_unsupported_codec_parameters_are_rejected():
    from superl8.quant import lloydmax

    with pytest.raises(ValueError):
        lloydmax.quantize_lloydmax(torch.zeros(1, 128), bits=4)
    with pytest.raises(ValueError):
        lloydmax.quantize_lloydmax(torch.zeros(1, 128), block_size=64)
    with pytest.raises(ValueError):
        lloydmax.quantize_lloydmax(torch.zeros(1, 128), dim=0)


_GUIDE = "INTEGRATION.md"  # the maintainer's binding guide at the repository root


def _integration_calls():
    """Every ``superl8.X`` / ``ops.X`` attribute named in the binding
    guide's Python code blocks (comments included: they show calls too)."""
    import re

    text = (Path(__file__).resolve().parent.parent / _GUIDE).read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    names = set()
    for blk in blocks:
        names.update(re.findall(r"\b((?:superl8|ops)(?:\.[A-Za-z_][A-Za-z_0-9]*)+)", blk))
    return sorted(names)


def test_integration_examples_name_only_real_functions():
    import superl8

    from superl8_serve_amd import ops

    names = _integration_calls()
    assert any(n.startswith("superl8.attn_paged_verify") for n in names)
    for name in names:
        root, *attrs = name.split(".")
        obj = superl8 if root == "superl8" else ops
        for attr in attrs:
            assert hasattr(obj, attr), f"the binding guide calls {name}, which does not resolve"
            obj = getattr(obj, attr)
        assert callable(obj) or inspect.ismodule(obj), name


@pytest.mark.parametrize("name", ["attn_paged_decode_append", "attn_paged_decode_append_k8v3",
                                  "attn_paged_decode_plan", "attn_paged_verify", "attn_paged_verify_k8v3",
                                  "attn_paged_decode_window", "attn_paged_decode_window_k8v3",
                                  "quantize_kv_write_paged_k8v3", "copy_blocks"])
def test_one_launch_ops_are_on_the_superl8_module(name):
    import superl8

    from superl8_serve_amd import ops

    assert getattr(superl8, name) is getattr(ops, name)
