"""Restatement of the part of KURN's API that COMP's verification calls -- TEST INFRASTRUCTURE ONLY.

KURN (the `kurn` package: exact references, test data, spec parsing) is a dependency of the reference that is neither
vendored in it nor installed here, and it is unversioned (pyproject.toml:13 lists plain "kurn").  comp_amd.verify, like
the reference's src/komp/verify.py:23-24, imports `kurn.formats` and `kurn.gpu.ref`; the tests put this directory on
sys.path so that those imports resolve to the restatement below, built on oracle/oracle.py.

Only the call sites in the reference pin this API (src/komp/verify.py:59,65,74,79,84-85,90,107,126,130,133,135 and
tests/test_komp.py:72-75).  The random streams and the "extreme" distributions of kurn.gpu.ref are KURN's own and
cannot be reproduced: these use this repository's seeded generators.  kurn.gpu.ref.relerr's formula is unknown
(parity unpinned): this one is the norm-wise max|y - r| / max|r|.
"""
