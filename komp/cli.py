"""`komp.cli` is `comp_amd.cli`: this module replaces itself with it on import."""

import sys

from comp_amd import cli as _module

sys.modules[__name__] = _module
