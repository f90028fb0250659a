"""soupsuck_amd: MI355X-native (gfx950 HIP) QLoRA NF4 hot path with the reference's API.

``apply()`` mirrors the reference's solution.apply() (solution/__init__.py:16-20):
an idempotent, lazy registration of the patches; no GPU work happens here.
"""

__all__ = ["apply"]


def apply():
    """Register patches lazily; repeated calls leave installed methods intact."""
    from .patch import install

    install()
