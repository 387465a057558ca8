"""`komp.verify` is `comp_amd.verify`: this module replaces itself with it on import."""

import sys

from comp_amd import verify as _module

sys.modules[__name__] = _module
