"""`komp.spec` is `comp_amd.spec`: this module replaces itself with it on import."""

import sys

from comp_amd import spec as _module

sys.modules[__name__] = _module
