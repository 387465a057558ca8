"""`komp.host` is `comp_amd.host`: this module replaces itself with it on import."""

import sys

from comp_amd import host as _module

sys.modules[__name__] = _module
