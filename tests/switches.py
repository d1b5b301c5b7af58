"""Kernel-selection switches of libc3hip.so for tests that compare two
kernels of one operation (C3H_DISABLE_DMA, C3H_DISABLE_BIGTILE, ...)."""

from __future__ import annotations

import os


def with_switch(var, value, fn):
    """Run `fn` with switch `var` set to `value` (None: unset); the library
    re-reads its switches on each change."""
    from hackathon_amd import _lib

    old = os.environ.get(var)
    if value is None:
        os.environ.pop(var, None)
    else:
        os.environ[var] = value
    _lib.check(_lib.lib().c3h_reload_switches(), "c3h_reload_switches")
    try:
        return fn()
    finally:
        if old is None:
            os.environ.pop(var, None)
        else:
            os.environ[var] = old
        _lib.check(_lib.lib().c3h_reload_switches(), "c3h_reload_switches")
