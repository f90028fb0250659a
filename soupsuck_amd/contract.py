"""Argument contracts of the drop-in entry points.

Every public entry point checks its arguments against an ordered table of
rules before it launches anything and raises ValueError carrying the first
broken rule's text; callers fall back to their original code on ValueError,
which is the reference's error behaviour (solution/nf4_patch.py:72-83).
Kernel failures are RuntimeError from the library and are never caught here.

A rule is ``(text, predicate)``; the predicate sees the entry point's
arguments as attributes of one namespace.  The tables are data, so which
inputs an entry point accepts can be read in one place per entry point.  The
few words the reference's tests match in these messages ("fp16", "state2",
"contiguous", "out_dtype", "CUDA", "2-D") appear in the corresponding texts.
"""

import math
import numbers
from types import SimpleNamespace
from typing import Callable, NamedTuple

import torch

FLOAT_DTYPES = (torch.float16, torch.float32)


class Rule(NamedTuple):
    text: str
    holds: Callable[[SimpleNamespace], bool]


def enforce(rules, **arguments):
    """Raise ValueError(text) for the first rule whose predicate is false."""
    ns = SimpleNamespace(**arguments)
    for rule in rules:
        if not rule.holds(ns):
            raise ValueError(rule.text)
    return ns


# ------------------------------------------------------------- predicates ---

def is_tensor(*values):
    return all(isinstance(v, torch.Tensor) for v in values)


def on_one_cuda_device(*tensors):
    """All are CUDA tensors on the first one's device (None entries are skipped)."""
    present = [t for t in tensors if t is not None]
    if not present or not is_tensor(*present) or not present[0].is_cuda:
        return False
    return all(t.device == present[0].device for t in present)


def float_dtypes(*tensors):
    return all(t.dtype in FLOAT_DTYPES for t in tensors if t is not None)


def finite_real(value, minimum=None):
    if isinstance(value, bool) or not isinstance(value, numbers.Real):
        return False
    if not math.isfinite(value):
        return False
    return minimum is None or value >= minimum


def frozen_buffer(t, dtype, device, at_least):
    """A contiguous, gradient-free tensor of ``dtype`` on ``device`` with >= at_least elements."""
    return (isinstance(t, torch.Tensor) and t.device == device and t.dtype == dtype
            and t.is_contiguous() and not t.requires_grad and t.numel() >= at_least)


def cdiv(a, b):
    return -(-a // b)
