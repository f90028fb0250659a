"""Runtime switches (reference solution/utils.py:6-8)."""

import os


def enabled():
    """Master switch: SOUP_FUSED_DISABLE=1/true/yes routes every patched entry to its original."""
    return os.environ.get("SOUP_FUSED_DISABLE", "0").lower() not in {"1", "true", "yes"}
