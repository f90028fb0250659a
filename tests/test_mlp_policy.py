"""Host logic of the MLP activation placement (no GPU): the per-layer policy of
the reference's solution/mlp.py:362-431 (SOUP_MLP_RECOMPUTE_LAYERS,
SOUP_EXP_OFFLOAD_TAIL, layer numbering by first run or by prepare_mlp_offload)
and the pinned pool's capacity classes."""

import pytest
import torch

from soupsuck_amd import mlp as fmlp


class _Cfg:
    hidden_act = "silu"

    def __init__(self, layers=None):
        if layers is not None:
            self.num_hidden_layers = layers


class _Stub(torch.nn.Module):
    """Only what the policy reads: the three projection names and a config."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        for name, (i, o) in {"gate_proj": (8, 24), "up_proj": (8, 24),
                             "down_proj": (24, 8)}.items():
            setattr(self, name, torch.nn.Linear(i, o, bias=False))


def test_capacity_classes():
    assert [fmlp._capacity(r) for r in (0, 1, 64, 65, 128, 129, 990, 1024, 1025)] == \
        [64, 64, 64, 128, 128, 256, 1024, 1024, 2048]


def test_layer_index_follows_first_run_order_per_config(monkeypatch):
    monkeypatch.setenv("SOUP_MLP_RECOMPUTE_LAYERS", "2")
    cfg, other = _Cfg(4), _Cfg(4)
    a, b, c, d = (_Stub(cfg) for _ in range(4))
    e = _Stub(other)
    # First calls number the layers of one config 0, 1, 2 ...; repeats keep theirs.
    assert [fmlp._layer_index(m) for m in (b, a, b, c, d, a)] == [0, 1, 0, 2, 3, 1]
    assert fmlp._layer_index(e) == 0
    assert [fmlp._recompute_layer(m) for m in (b, a, c, d, e)] == [True, True, False, False,
                                                                   True]


def test_env_values_are_checked_against_the_depth(monkeypatch):
    layer = _Stub(_Cfg(3))
    for value in ("-1", "4", "x"):
        monkeypatch.setenv("SOUP_MLP_RECOMPUTE_LAYERS", value)
        with pytest.raises(ValueError, match="SOUP_MLP_RECOMPUTE_LAYERS"):
            fmlp._recompute_layer(layer)
    monkeypatch.setenv("SOUP_MLP_RECOMPUTE_LAYERS", "3")
    assert fmlp._recompute_layer(layer)
    monkeypatch.setenv("SOUP_EXP_OFFLOAD_TAIL", "4")
    with pytest.raises(ValueError, match="SOUP_EXP_OFFLOAD_TAIL"):
        fmlp._tail_layer(layer)
    # Without a known depth the tail cannot be placed.
    monkeypatch.setenv("SOUP_EXP_OFFLOAD_TAIL", "1")
    with pytest.raises(ValueError, match="prepare_mlp_offload"):
        fmlp._tail_layer(_Stub(_Cfg()))
    monkeypatch.setenv("SOUP_EXP_OFFLOAD_TAIL", "0")
    assert not fmlp._tail_layer(_Stub(_Cfg()))


def test_prepare_numbers_layers_in_module_order(monkeypatch):
    model = torch.nn.ModuleList([_Stub(_Cfg()) for _ in range(5)])
    monkeypatch.setenv("SOUP_MLP_RECOMPUTE_LAYERS", "2")
    monkeypatch.setenv("SOUP_EXP_OFFLOAD_TAIL", "2")
    # CPU modules: numbered, nothing reserved.
    assert fmlp.prepare_mlp_offload(model, max_rows=128) == 5
    assert [m._soup_mlp_index for m in model] == [0, 1, 2, 3, 4]
    assert [fmlp._recompute_layer(m) for m in model] == [True, True, False, False, False]
    assert [fmlp._tail_layer(m) for m in model] == [False, False, False, True, True]
    with pytest.raises(ValueError):
        fmlp.prepare_mlp_offload(model, max_rows=0)
