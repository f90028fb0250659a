"""Runtime switches (reference solution/utils.py:6-8) and the hook check the routes share."""

import os

# Attribute carried by a per-instance forward this package installs itself (the
# packed-layout LoRA dropout of soupsuck_amd.unpad_route); it names the original.
BOUND_MARKER = "_soupsuck_bound_original"


def enabled():
    """Master switch: SOUP_FUSED_DISABLE=1/true/yes routes every patched entry to its original."""
    return os.environ.get("SOUP_FUSED_DISABLE", "0").lower() not in {"1", "true", "yes"}


def hookless(*modules):
    """No forward / backward hooks and no per-instance forward on any module, except a
    forward this package bound (marked with BOUND_MARKER)."""
    for m in modules:
        if (m._forward_hooks or m._forward_pre_hooks or m._backward_hooks
                or getattr(m, "_backward_pre_hooks", None)):
            return False
        own = m.__dict__.get("forward")
        if own is not None and not hasattr(own, BOUND_MARKER):
            return False
    return True
