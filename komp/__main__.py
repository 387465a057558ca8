"""`python -m komp ...`: comp_amd's command line (the reference's src/komp/__main__.py)."""

import sys

from comp_amd.cli import main

sys.exit(main())
