"""soupsuck_amd: MI355X-native (gfx950 HIP) QLoRA NF4 hot path with the reference's API.

``apply()`` mirrors the reference's solution.apply() (solution/__init__.py:16-20):
an idempotent, lazy registration of the routes (soupsuck_amd.patch); no GPU work
happens here.  When no bitsandbytes is importable (as on this ROCm image) it also
registers soupsuck_amd.bnb_compat under the ``bitsandbytes`` import names, unless
SOUP_BNB_COMPAT=0.
"""

import os

__all__ = ["apply"]


def apply():
    """Register routes lazily; repeated calls leave installed methods intact."""
    from .patch import install

    if os.environ.get("SOUP_BNB_COMPAT", "1").lower() not in {"0", "false", "no"}:
        from .bnb_compat import register_as_bitsandbytes

        register_as_bitsandbytes()
    install()
