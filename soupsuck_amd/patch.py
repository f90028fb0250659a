"""Lazy, idempotent routing of the reference's patch surface (solution/patch.py:441-487).

A *route* replaces one function or method of a third-party module by a
version that sends supported calls to this package's HIP path and every other
call to the original.  Routes are declared as data (``ROUTES``): the module
name, the owning class (or None for a module attribute), the attribute, the
builder that makes the replacement from the original, and the marker
attribute that holds the original.  ``install()`` installs the routes of
modules already imported and puts one ``sys.meta_path`` finder in front that
installs the others as soon as their module is imported, so the order of
``apply()`` and the imports does not matter.  No GPU work happens here.

Routes (reference file of the behaviour each one keeps):
  bitsandbytes 0.50.2 (solution/nf4_patch.py:43-125), in soupsuck_amd.bnb_routes:
    functional.dequantize_4bit, backends.cuda.ops._dequantize_4bit_impl and
    _dequant_linear_fallback, and matmul_4bit (the NF4 GEMM);
  transformers Qwen2 (modeling_qwen2):
    Qwen2DecoderLayer.forward  attention residual add + post-attention norm
                               fused (solution/decoder.py:54-89), with the fp16
                               norm-output scopes of soupsuck_amd.norm_scope;
    Qwen2RMSNorm.forward       the HIP row norm, fp16 output for the scoped owner
                               (solution/patch.py:35-125,232-250);
    Qwen2MLP.forward           the frozen NF4 MLP node (solution/mlp.py:597-612);
    apply_rotary_pos_emb       the joint q/k RoPE (solution/rope.py:55-80);
    Qwen2ForCausalLM.forward   the chunked fused CE head (solution/patch.py:167-229),
                               in soupsuck_amd.head;
    Qwen2Model.forward,        right-padded batches packed to their real tokens,
    Qwen2Attention.forward     causal attention within each row in one launch
                               (solution/unpad.py:359-450), in soupsuck_amd.unpad_route;
  PEFT (solution/lora.py:135-166), in soupsuck_amd.peft_route:
    tuners.lora.bnb.Linear4bit.forward  the fused QLoRA projection;
  Soup (solution/embedding.py:146-169), in soupsuck_amd.embedding:
    trainer.sft.SFTTrainerWrapper._setup_transformers  lossless fp16 storage of the
                               tied embedding / lm_head after the original setup.
Every replacement falls back to the original when SOUP_FUSED_DISABLE is set
or a call is outside the supported contract, and carries the original under
its marker (``_solution_fused_original``; the PEFT route uses
``_solution_lora_4bit_original``, as the reference does).
"""

import functools
import importlib
import sys
from importlib.abc import Loader, MetaPathFinder
from importlib.machinery import PathFinder
from types import ModuleType
from typing import Callable, NamedTuple, Optional

from .utils import enabled

MARKER = "_solution_fused_original"
QWEN = "transformers.models.qwen2.modeling_qwen2"


class Route(NamedTuple):
    module: str
    owner: Optional[str]                 # class in ``module``; None for a module attribute
    attr: str
    build: Callable                      # build(original, module) -> replacement or None
    marker: str = MARKER


def _holder(route, module):
    if route.owner is None:
        return module
    cls = getattr(module, route.owner, None)
    return cls if isinstance(cls, type) else None


def install_route(route, module=None):
    """Install one route on ``module`` (imported if None); True when it is in place."""
    if module is None:
        try:
            module = importlib.import_module(route.module)
        except (ImportError, AttributeError):
            return False
    if not isinstance(module, ModuleType):
        return False
    holder = _holder(route, module)
    original = getattr(holder, route.attr, None) if holder is not None else None
    if not callable(original):
        return False
    if hasattr(original, route.marker):
        return True
    replacement = route.build(original, module)
    if replacement is None:
        return False
    functools.update_wrapper(replacement, original)
    setattr(replacement, route.marker, original)
    setattr(holder, route.attr, replacement)
    return True


# ---------------------------------------------------------------- Qwen2 ---

def _float_cuda(t):
    import torch

    return (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype in (torch.float16, torch.float32)
            and t.is_contiguous())


def _hookless(module):
    return not (module._forward_hooks or module._forward_pre_hooks)


def _exact_class(module, name):
    cls = getattr(module, name, None)
    if not isinstance(cls, type) or cls.__module__ != module.__name__:
        return None
    return cls


# Qwen2DecoderLayer.forward's arguments after hidden_states, with their defaults.
_DECODER_ARGS = (("attention_mask", None), ("position_ids", None), ("past_key_values", None),
                 ("use_cache", False), ("position_embeddings", None))


def _residual_norm(norm, norm_cls, residual, update, half=False):
    """(residual + update, norm(residual + update)); one HIP pass when the norm qualifies,
    with an fp16 norm output when ``half`` (the layer's MLP consumes it as fp16)."""
    weight = getattr(norm, "weight", None)
    if (type(norm) is norm_cls and _hookless(norm) and _float_cuda(update) and _float_cuda(weight)
            and update.shape == residual.shape and weight.ndim == 1
            and weight.numel() == residual.shape[-1]
            and update.device == residual.device == weight.device):
        import torch

        from .kernels.add_rmsnorm import add_rms_norm

        return add_rms_norm(residual, update, weight, norm.variance_epsilon,
                            torch.float16 if half else None)
    total = residual + update
    return total, norm(total)


def _build_decoder(original, module):
    cls, norm_cls = _exact_class(module, "Qwen2DecoderLayer"), _exact_class(module, "Qwen2RMSNorm")
    if cls is None or norm_cls is None:
        return None

    def forward(self, hidden_states, *args, **kwargs):
        if not enabled() or type(self) is not cls or not _float_cuda(hidden_states) \
                or len(args) > len(_DECODER_ARGS):
            return original(self, hidden_states, *args, **kwargs)
        named = dict(zip((name for name, _ in _DECODER_ARGS), args))
        if set(named) & set(kwargs):
            return original(self, hidden_states, *args, **kwargs)
        call = dict(_DECODER_ARGS)
        call.update(named)
        call.update(kwargs)
        from .norm_scope import half_norm_scope, input_norm_half_ready, post_norm_half_ready

        owner = self.input_layernorm if input_norm_half_ready(self, hidden_states, kwargs) \
            else None
        with half_norm_scope(owner):
            normed = self.input_layernorm(hidden_states)
        attended, _ = self.self_attn(hidden_states=normed, **call)
        residual, normed = _residual_norm(self.post_attention_layernorm, norm_cls,
                                          hidden_states, attended,
                                          post_norm_half_ready(self, hidden_states))
        return residual + self.mlp(normed)

    return forward


def _build_rmsnorm(original, module):
    cls = _exact_class(module, "Qwen2RMSNorm")
    if cls is None:
        return None

    def forward(self, hidden_states):
        weight = getattr(self, "weight", None)
        if (enabled() and type(self) is cls and _hookless(self) and _float_cuda(hidden_states)
                and _float_cuda(weight) and weight.ndim == 1
                and weight.shape[0] == hidden_states.shape[-1]
                and weight.device == hidden_states.device):
            import torch

            from .kernels.rmsnorm import rms_norm
            from .norm_scope import owns_half_output

            half = torch.float16 if owns_half_output(self) else None
            return rms_norm(hidden_states, weight, self.variance_epsilon, half)
        return original(self, hidden_states)

    return forward


def _build_mlp(original, module):
    cls = _exact_class(module, "Qwen2MLP")
    if cls is None:
        return None
    from .mlp import eligible_mlp, fused_qwen2_mlp

    def forward(self, x):
        if enabled() and type(self) is cls and eligible_mlp(self, x):
            return fused_qwen2_mlp(self, x)
        return original(self, x)

    return forward


def _build_rope(original, module):
    from .kernels.rope import fused_rope, rope_supported

    def apply_rotary_pos_emb(q, k, cos, sin, *args, **kwargs):
        dim = kwargs.get("unsqueeze_dim", 1)
        if args or not enabled() or not rope_supported(q, k, cos, sin, dim):
            return original(q, k, cos, sin, *args, **kwargs)
        return fused_rope(q, k, cos, sin)

    return apply_rotary_pos_emb


def _build_head(original, module):
    from .head import build_causal_lm_forward

    return build_causal_lm_forward(original, module)


def _build_model(original, module):
    from .unpad_route import build_model_forward

    return build_model_forward(original, module)


def _build_attention(original, module):
    from .unpad_route import build_attention_forward

    return build_attention_forward(original, module)


def _build_bnb(name):
    def build(original, module):
        from . import bnb_routes

        return getattr(bnb_routes, name)(original, module)

    return build


def _build_soup_setup(original, module):
    from .embedding import build_soup_setup

    return build_soup_setup(original, module)


def _build_peft(original, module):
    from .peft_route import build_linear4bit_forward

    return build_linear4bit_forward(original, module)


DECODER_ROUTE = Route(QWEN, "Qwen2DecoderLayer", "forward", _build_decoder)
RMSNORM_ROUTE = Route(QWEN, "Qwen2RMSNorm", "forward", _build_rmsnorm)
MLP_ROUTE = Route(QWEN, "Qwen2MLP", "forward", _build_mlp)
ROPE_ROUTE = Route(QWEN, None, "apply_rotary_pos_emb", _build_rope)
HEAD_ROUTE = Route(QWEN, "Qwen2ForCausalLM", "forward", _build_head)
MODEL_ROUTE = Route(QWEN, "Qwen2Model", "forward", _build_model)
ATTENTION_ROUTE = Route(QWEN, "Qwen2Attention", "forward", _build_attention)
PEFT_ROUTE = Route("peft.tuners.lora.bnb", "Linear4bit", "forward", _build_peft,
                   "_solution_lora_4bit_original")
SOUP_SETUP_ROUTE = Route("soup_cli.trainer.sft", "SFTTrainerWrapper", "_setup_transformers",
                         _build_soup_setup)
BNB_ROUTES = (
    Route("bitsandbytes.functional", None, "dequantize_4bit", _build_bnb("build_dequantize")),
    Route("bitsandbytes.backends.cuda.ops", None, "_dequantize_4bit_impl",
          _build_bnb("build_backend_decode")),
    Route("bitsandbytes.backends.cuda.ops", None, "_dequant_linear_fallback",
          _build_bnb("build_linear_fallback")),
    Route("bitsandbytes", None, "matmul_4bit", _build_bnb("build_matmul")),
)
ROUTES = (DECODER_ROUTE, RMSNORM_ROUTE, MLP_ROUTE, ROPE_ROUTE, HEAD_ROUTE, MODEL_ROUTE,
          ATTENTION_ROUTE, PEFT_ROUTE, SOUP_SETUP_ROUTE) + BNB_ROUTES
TARGETS = tuple(sorted({r.module for r in ROUTES}))


def patch_qwen2_decoder(module=None):
    return install_route(DECODER_ROUTE, module)


def patch_qwen2_rmsnorm(module=None):
    return install_route(RMSNORM_ROUTE, module)


def patch_qwen2_head(module=None):
    return install_route(HEAD_ROUTE, module)


def patch_qwen2_unpad(module=None):
    return [install_route(MODEL_ROUTE, module), install_route(ATTENTION_ROUTE, module)]


def patch_peft_linear4bit(module=None):
    return install_route(PEFT_ROUTE, module)


def patch_bnb(modules=None):
    """Install the bitsandbytes routes; ``modules`` maps module names to (fake) modules."""
    modules = modules or {}
    return [install_route(r, modules.get(r.module)) for r in BNB_ROUTES]


def routes_for(module):
    """Install the routes of ``module`` and of its loaded submodules (called right after
    it is imported: a package's submodules may load while the package itself is still
    initialising, before the attributes a builder checks, such as __version__, exist)."""
    name = module.__name__
    for route in ROUTES:
        if route.module == name:
            install_route(route, module)
        elif route.module.startswith(name + ".") and route.module in sys.modules:
            install_route(route, sys.modules[route.module])


class _RoutingLoader(Loader):
    def __init__(self, loader):
        self.loader = loader

    def create_module(self, spec):
        return self.loader.create_module(spec)

    def exec_module(self, module):
        self.loader.exec_module(module)
        routes_for(module)


class _RoutingFinder(MetaPathFinder):
    _solution_patch_finder = True

    def find_spec(self, fullname, path, target=None):
        if fullname not in TARGETS:
            return None
        spec = PathFinder.find_spec(fullname, path)
        if spec is None or spec.loader is None:
            return None
        spec.loader = _RoutingLoader(spec.loader)
        return spec


def install():
    """Idempotent: one finder on sys.meta_path; routes of imported targets installed now."""
    if not any(getattr(f, "_solution_patch_finder", False) for f in sys.meta_path):
        sys.meta_path.insert(0, _RoutingFinder())
    for name in TARGETS:
        module = sys.modules.get(name)
        if module is not None:
            routes_for(module)
