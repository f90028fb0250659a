"""Unpadded decoder stack: Qwen2Model runs right-padded batches as one packed row set.

Behaviour of the reference's unpad path (solution/unpad.py:164-199,413-450):
a right-padded batch [B, S] is packed to its T real tokens [1, T] before the
decoder layers (no padding rows in any projection, norm or MLP), attention
runs causally within each original row (solution/unpad.py:359-410), and the
final hidden states are scattered back to [B, S, H] with zero padding rows.

Here the pieces are this package's kernels: ss_unpad_gather / ss_unpad_scatter
for packing, and ss_attn_varlen_fwd / _bwd (kernels/attention.py) for the
attention of all rows and heads in one launch, instead of one SDPA call per
row.  The causal-LM head route reads the packed hidden states that this route
publishes and runs the fused cross-entropy on the real rows only
(soupsuck_amd.head).

When a batch packs is the ordered guard table GUARDS below (a failed guard
runs the original forward; ``last_refusal()`` names it), followed by one
device-to-host check that the mask is binary and right-padded with at least
one padding position and, when the head passes labels, that every padding
position is labelled -100.

Dropout.  Packing changes the layout a dropout draws its mask over, so an
active torch Dropout anywhere in the model refuses packing -- except the LoRA
dropouts of PEFT ``Linear4bit`` layers that carry this package's PEFT route
(the reference likewise certifies its q/v adapter dropouts,
solution/unpad.py:207-273).  Such a layer's routed call never runs the module:
its keep mask is the fused Philox mask of soupsuck_amd.lora, drawn per packed
element.  If a call of the layer falls back to PEFT's own forward instead,
the module runs bound to the packed batch: its input is scattered to the
padded layout, the module's original forward runs there once and the result
is packed again, so torch's RNG draws exactly the masks of the padded run
(the reference's binding, solution/unpad.py:325-345).
"""

import os
from contextvars import ContextVar
from types import MethodType, SimpleNamespace
from typing import Callable, NamedTuple

import torch

from .utils import BOUND_MARKER, enabled
from .utils import hookless as _hookless

_PACKED = ContextVar("soupsuck_packed_batch", default=None)
HEAD_LABELS = ContextVar("soupsuck_head_labels", default=None)
_REFUSAL = ContextVar("soupsuck_unpad_refusal", default=None)
_ALLOWED_KWARGS = ("num_items_in_batch", "output_hidden_states", "output_attentions",
                   "return_dict")
_PROJECTIONS = (("self_attn", ("q_proj", "k_proj", "v_proj", "o_proj")),
                ("mlp", ("gate_proj", "up_proj", "down_proj")))


def unpad_enabled():
    return enabled() and os.environ.get("SOUP_UNPAD", "1").lower() not in {"0", "false", "no"}


def last_refusal():
    """The guard text that last kept a Qwen2Model call unpacked in this context, or None."""
    return _REFUSAL.get()


# ------------------------------------------------------------ dropouts ---

def _routed_lora(projection):
    """The active adapter's dropout module of a PEFT Linear4bit routed by this package, else
    None.  The class must carry the PEFT route (its forward is this package's)."""
    from .patch import PEFT_ROUTE

    cls = type(projection)
    if cls.__name__ != PEFT_ROUTE.owner or not hasattr(cls.forward, PEFT_ROUTE.marker):
        return None
    active = getattr(projection, "active_adapters", None)
    dropouts = getattr(projection, "lora_dropout", None)
    if not active or len(active) != 1 or dropouts is None or active[0] not in dropouts:
        return None
    return dropouts[active[0]]


def _active(module):
    return isinstance(module, torch.nn.Dropout) and module.training and module.p


def packable_dropouts(model):
    """frozenset of the ids of the active LoRA dropouts packing keeps, or None when some
    active Dropout would see the packed layout through torch's RNG (see the module text)."""
    if not model.training:
        return frozenset()
    accepted = {}
    for layer in model.layers:
        for owner, names in _PROJECTIONS:
            parent = getattr(layer, owner, None)
            for name in names:
                drop = _routed_lora(getattr(parent, name, None))
                if drop is None or not _active(drop):
                    continue
                if (type(drop) is not torch.nn.Dropout or drop.inplace
                        or not _hookless(drop)):
                    return None
                accepted[id(drop)] = drop
    for child in model.modules():
        if _active(child) and id(child) not in accepted:
            return None
    for drop in accepted.values():
        _bind_dropout(drop)
    return frozenset(accepted)


def _bind_dropout(drop):
    """Run ``drop`` on the padded layout whenever it sees a packed batch it belongs to."""
    own = drop.__dict__.get("forward")
    if own is not None and hasattr(own, BOUND_MARKER):
        return
    original = drop.forward

    def forward(self, x):
        batch = _PACKED.get()
        if batch is None or id(self) not in batch.dropout_ids:
            return original(x)
        if x.numel() != batch.tokens * x.shape[-1]:
            raise RuntimeError("a packed LoRA dropout saw an input that is not the packed batch")
        from .unpad import pack, scatter

        padded = scatter(x.reshape(1, batch.tokens, x.shape[-1]), batch)
        return pack(original(padded), batch).reshape(x.shape)

    setattr(forward, BOUND_MARKER, original)
    drop.forward = MethodType(forward, drop)


# -------------------------------------------------------------- guards ---

class Guard(NamedTuple):
    text: str
    holds: Callable[[SimpleNamespace], bool]


def _layers_packable(c):
    for layer in c.model.layers:
        attn = getattr(layer, "self_attn", None)
        if (type(layer) is not c.module.Qwen2DecoderLayer
                or type(attn) is not c.module.Qwen2Attention or not _hookless(attn)
                or attn.head_dim != 128 or getattr(attn, "sliding_window", None) is not None
                or (c.model.training and attn.attention_dropout)):
            return False
    return True


def _source(c):
    return c.input_ids if c.input_ids is not None else c.inputs_embeds


def _fp16_compute(c):
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16:
        return True
    embed = c.model.embed_tokens.weight if c.input_ids is not None else c.inputs_embeds
    return embed.dtype == torch.float16


def _positions_fit(c):
    p, mask = c.position_ids, c.attention_mask
    return p is None or (isinstance(p, torch.Tensor) and p.ndim == 2
                         and p.shape[1] == mask.shape[1] and p.shape[0] in (1, mask.shape[0]))


def _kwargs_fit(c):
    kw = c.kwargs
    return (all(k in _ALLOWED_KWARGS for k in kw) and not kw.get("output_hidden_states")
            and not kw.get("output_attentions") and kw.get("return_dict") is not False)


def _cache_off(c):
    cache = c.use_cache if c.use_cache is not None else getattr(c.model.config, "use_cache",
                                                                False)
    return c.past_key_values is None and not cache


def _dropouts_fit(c):
    c.dropout_ids = packable_dropouts(c.model)
    return c.dropout_ids is not None


GUARDS = (
    Guard("packing is off (SOUP_FUSED_DISABLE=1 or SOUP_UNPAD=0)", lambda c: unpad_enabled()),
    Guard("the model is not an exact, hook-free Qwen2Model",
          lambda c: type(c.model) is c.module.Qwen2Model and _hookless(c.model)),
    Guard("a packed batch is already running", lambda c: _PACKED.get() is None),
    Guard("a KV cache is in use", _cache_off),
    Guard("gradient checkpointing is on",
          lambda c: not getattr(c.model, "gradient_checkpointing", False)),
    Guard("the model has sliding-window layers",
          lambda c: not getattr(c.model, "has_sliding_layers", False)),
    Guard("the rotary embedding is not the default one",
          lambda c: getattr(c.model.rotary_emb, "rope_type", "default") == "default"),
    Guard("keyword arguments other than num_items_in_batch, falsy output_* and return_dict",
          _kwargs_fit),
    Guard("the attention mask is not a 2-D tensor without gradient",
          lambda c: isinstance(c.attention_mask, torch.Tensor) and c.attention_mask.ndim == 2
          and not c.attention_mask.requires_grad),
    Guard("exactly one of input_ids and inputs_embeds must be given",
          lambda c: (c.input_ids is None) != (c.inputs_embeds is None)),
    Guard("the inputs are not CUDA tensors of the mask's [B, S] on its device",
          lambda c: isinstance(_source(c), torch.Tensor) and _source(c).is_cuda
          and _source(c).shape[:2] == c.attention_mask.shape
          and _source(c).device == c.attention_mask.device),
    Guard("the model does not compute in fp16 (fp16 autocast or fp16 embeddings)",
          _fp16_compute),
    Guard("position_ids is not [1 or B, S]", _positions_fit),
    Guard("a layer is not an exact Qwen2DecoderLayer over a hook-free Qwen2Attention with "
          "head_dim 128, full attention and no attention dropout", _layers_packable),
    Guard("an active Dropout other than a routed PEFT Linear4bit's LoRA dropout",
          _dropouts_fit),
)


def right_padded_lengths(attention_mask, labels):
    """Row lengths of a binary right-padded mask whose padding labels are -100, else None.

    One device-to-host transfer carries the mask and the validity flag."""
    from .unpad import right_padding_lengths

    real = attention_mask != 0
    ok = ((attention_mask == 0) | (attention_mask == 1)).all()
    if labels is not None:
        ok = ok & (real | (labels == -100)).all()
    flat = torch.cat((real.reshape(-1).to(torch.uint8), ok.reshape(1).to(torch.uint8)))
    values = flat.tolist()
    if not values[-1]:
        return None
    s = attention_mask.shape[1]
    return right_padding_lengths([values[i:i + s] for i in range(0, len(values) - 1, s)])


def plan(model, module, input_ids, attention_mask, position_ids, past_key_values, inputs_embeds,
         use_cache, kwargs):
    """The PackedBatch to run ``model`` on, or None to run the original forward."""
    c = SimpleNamespace(model=model, module=module, input_ids=input_ids,
                        attention_mask=attention_mask, position_ids=position_ids,
                        past_key_values=past_key_values, inputs_embeds=inputs_embeds,
                        use_cache=use_cache, kwargs=kwargs, dropout_ids=None)
    for guard in GUARDS:
        if not guard.holds(c):
            _REFUSAL.set(guard.text)
            return None
    labels = HEAD_LABELS.get()
    if labels is not None and (labels[1] is not attention_mask
                               or labels[0].shape != attention_mask.shape):
        labels = None
    lengths = right_padded_lengths(attention_mask, None if labels is None else labels[0])
    b, s = attention_mask.shape
    if lengths is None or sum(lengths) == b * s:
        _REFUSAL.set("the mask is not binary right padding with at least one padding position "
                     "(or a padding position has a label other than -100)")
        return None
    from .kernels.attention import row_offsets
    from .unpad import make_batch

    source = _source(c)
    batch = make_batch(lengths, s, source.device)
    batch.cu_seqlens = row_offsets(lengths, source.device)
    batch.attention_ids = frozenset(id(layer.self_attn) for layer in model.layers)
    batch.dropout_ids = c.dropout_ids
    _REFUSAL.set(None)
    return batch


def build_model_forward(original, module):
    cls = getattr(module, "Qwen2Model", None)
    if not isinstance(cls, type):
        return None

    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, use_cache=None, **kwargs):
        args = dict(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                    past_key_values=past_key_values, inputs_embeds=inputs_embeds,
                    use_cache=use_cache, **kwargs)
        batch = plan(self, module, input_ids, attention_mask, position_ids, past_key_values,
                     inputs_embeds, use_cache, kwargs)
        if batch is None:
            return original(self, **args)
        from transformers.modeling_outputs import BaseModelOutputWithPast

        from .unpad import pack, scatter

        positions = position_ids
        if positions is None:
            positions = torch.arange(batch.sequence, device=batch.indices.device)[None]
        positions = positions.expand(batch.batch, batch.sequence).reshape(-1)
        packed_positions = positions.index_select(0, batch.indices)[None]
        packed_ids = pack(input_ids, batch) if input_ids is not None else None
        packed_embeds = pack(inputs_embeds, batch) if inputs_embeds is not None else None
        token = _PACKED.set(batch)
        try:
            out = original(self, input_ids=packed_ids, inputs_embeds=packed_embeds,
                           attention_mask={"full_attention": None},
                           position_ids=packed_positions, past_key_values=None,
                           use_cache=False, **kwargs)
        finally:
            _PACKED.reset(token)
        packed_hidden = out.last_hidden_state
        padded = scatter(packed_hidden, batch)
        self._soupsuck_packed_head = (batch, packed_hidden, padded)
        return BaseModelOutputWithPast(last_hidden_state=padded, past_key_values=None)

    return forward


def build_attention_forward(original, module):
    cls = getattr(module, "Qwen2Attention", None)
    if not isinstance(cls, type):
        return None

    def forward(self, hidden_states, position_embeddings, attention_mask=None,
                past_key_values=None, **kwargs):
        batch = _PACKED.get()
        if batch is None or id(self) not in batch.attention_ids:
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values=past_key_values, **kwargs)
        from .kernels.attention import packed_causal_attention

        shape = (*hidden_states.shape[:-1], -1, self.head_dim)
        q = self.q_proj(hidden_states).view(shape).transpose(1, 2)
        k = self.k_proj(hidden_states).view(shape).transpose(1, 2)
        v = self.v_proj(hidden_states).view(shape).transpose(1, 2)
        q, k = module.apply_rotary_pos_emb(q, k, *position_embeddings)
        out = packed_causal_attention(q.half(), k.half(), v.half(), batch.lengths, self.scaling,
                                      cu_seqlens=batch.cu_seqlens)
        out = out.reshape(*hidden_states.shape[:-1], -1)
        return self.o_proj(out), None

    return forward


def take_packed_head(model, hidden):
    """(batch, packed hidden) published by the model route for exactly this output, else None."""
    published = getattr(model, "_soupsuck_packed_head", None)
    model._soupsuck_packed_head = None
    if published is None or published[2] is not hidden:
        return None
    return published[0], published[1]
