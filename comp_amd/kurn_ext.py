"""KURN backend registration: `kurn check|verify SPEC` on a spec whose target is triton (or hip) runs this package.

The reference keeps this shim inside KURN (kurn/src/kurn/ext/komp.py:10-19).  Here it is a function a KURN build calls
with its hooks module, so the routing needs no file in KURN's tree beyond one call (see the integration notes)."""

from __future__ import annotations

import sys


def _spec_command(cmd, argv):
    try:
        from comp_amd.cli import spec_command
    except ImportError as e:  # the HIP package is optional for KURN
        print(f"kurn {cmd}: target triton needs the comp_amd package ({e})", file=sys.stderr)
        return 2
    return spec_command(cmd, argv)


def register(hooks):
    """Route KURN's `triton` and `hip` targets to comp_amd (kurn/src/kurn/ext/komp.py:19)."""
    hooks.TARGET_BACKENDS["triton"] = _spec_command
    hooks.TARGET_BACKENDS["hip"] = _spec_command
    return hooks.TARGET_BACKENDS
