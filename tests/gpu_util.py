"""Helpers shared by the GPU parity tests (host-side conversions only)."""

from types import SimpleNamespace

import numpy as np
import torch

from oracle import nf4 as onf4


def device_state(state, device):
    """QuantState-like namespace (bitsandbytes field names) from an oracle NF4State."""
    second = SimpleNamespace(
        blocksize=256, dtype=torch.float32, nested=False,
        code=torch.from_numpy(np.ascontiguousarray(state.code2)).to(device),
        absmax=torch.from_numpy(np.ascontiguousarray(state.absmax2)).to(device))
    packed = torch.from_numpy(np.ascontiguousarray(state.packed)).to(device).view(-1, 1)
    qs = SimpleNamespace(
        quant_type="nf4", blocksize=64, dtype=torch.float16, nested=True,
        shape=tuple(int(d) for d in state.shape),
        absmax=torch.from_numpy(np.ascontiguousarray(state.qabs)).to(device),
        state2=second,
        offset=torch.from_numpy(np.ascontiguousarray(state.offset)).to(device))
    return packed, qs


def random_weight(n, k, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, k), dtype=np.float32) * scale).astype(np.float16)


def quantized(n, k, seed):
    """(oracle state, decoded fp16 weight) of a seeded N(0, 0.02) weight."""
    state = onf4.quantize_nested(random_weight(n, k, seed))
    return state, state.decode()


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy()


def np16(t):
    return t.detach().cpu().numpy()


def rel_norm(actual, expected):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-300))
