"""Make ``import superl8`` resolve to this package's ``superl8`` interface.

The reference's cache code imports ``superl8`` and
``superl8.quant.rotation`` / ``superl8.quant.lloydmax`` at module level and at
call time (kv_cache.py:35-36, 502, 594, 613, 643, 1263).  ``install()``
registers ``superl8_serve_amd.superl8`` and its submodules under those names
in ``sys.modules``, so an unchanged ``kv_cache.py`` imported afterwards binds
to the gfx950 kernels."""

from __future__ import annotations

import sys
import types

_NAMES = ("superl8", "superl8.quant", "superl8.quant.rotation", "superl8.quant.lloydmax")


def install() -> types.ModuleType:
    """Register the modules; returns the ``superl8`` module.  Idempotent."""
    from . import superl8 as pkg
    from .superl8 import quant
    from .superl8.quant import lloydmax, rotation

    for name, mod in zip(_NAMES, (pkg, quant, rotation, lloydmax)):
        sys.modules[name] = mod
    return pkg


def installed() -> bool:
    """Whether ``import superl8`` currently resolves to this package."""
    from . import superl8 as pkg

    return sys.modules.get("superl8") is pkg
