"""`komp`, the import name the reference's callers use (pyproject.toml:6, src/komp/), for this build's decode path.

The modules are comp_amd's: `komp.host`, `komp.spec`, `komp.verify` and `komp.cli` are the comp_amd modules
themselves (the same module objects), so `from komp import host; host.gemv(...)` runs the gfx950 library, and
`python -m komp check|verify|gen|mix ...` or the `komp` console script (pyproject.toml) runs comp_amd's command line.
Importing `komp` alone loads nothing; each module loads when it is first imported."""

import importlib

_MODULES = ("host", "spec", "verify", "cli")


def __getattr__(name):
    if name in _MODULES:
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
