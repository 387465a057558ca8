"""KURN's backend registry (restated): target name -> callable(cmd, argv) -> exit code (kurn/src/kurn/ext/komp.py:19)."""

TARGET_BACKENDS = {}
