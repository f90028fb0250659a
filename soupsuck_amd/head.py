"""The fused causal-LM head: label shift, row selection, chunked CE, mean (A19 caller).

``fused_head`` follows the reference's solution/autograd.py:11-82:
  * targets are the labels shifted left by one inside the original [B, S]
    layout, the last column ignored (-100) -- the shift happens BEFORE any row
    selection, so the last real token of a short row predicts its padding,
    never the next row's first label;
  * with a packed batch (``packed``: a soupsuck_amd.unpad.PackedBatch and the
    packed hidden [1, T, H]) only the real positions go through the head: the
    shifted targets are gathered with the batch's indices;
  * loss = sum of per-token losses / denominator, the denominator being
    ``num_items_in_batch`` when the trainer gives one, else the number of
    labelled targets (the original mean's denominator either way);
  * detached per-token loss / entropy in the [B, S] layout (zero at padding)
    and the correct / labelled counts are returned for logging (the
    reference returns them in soup's ChunkedStep; soup is not part of this
    path, so a plain ``HeadStep`` carries the same fields).

``build_causal_lm_forward`` routes ``Qwen2ForCausalLM.forward`` (reference
solution/patch.py:167-229) to it when labels are given and the head is a
plain bias-free Linear on the hidden states' device; the model's logits are
then never materialised (``logits`` is None in the output).  When the model
route packed the batch (soupsuck_amd.unpad_route, which also checks that the
labels are -100 at every padding position), the head reads the packed hidden
states it published and runs on the real rows only.
"""

from dataclasses import dataclass

import torch

from .utils import enabled

IGNORE = -100


@dataclass
class HeadStep:
    token_loss: torch.Tensor      # [B, S] fp32, detached, zero where ignored
    token_entropy: torch.Tensor   # [B, S] fp32, detached
    correct: torch.Tensor         # scalar int64: argmax == target over labelled targets
    labelled: torch.Tensor        # scalar int64: number of labelled targets


def shift_targets(labels):
    """targets[..., t] = labels[..., t + 1]; the last position is ignored."""
    targets = torch.full_like(labels, IGNORE)
    if labels.shape[-1] > 1:
        targets[..., :-1] = labels[..., 1:]
    return targets


def select_targets(labels, indices=None):
    """Flat targets of the head rows: shifted in the [B, S] layout, then (packed)
    gathered at the real positions ``indices``."""
    flat = shift_targets(labels).reshape(-1)
    return flat if indices is None else flat.index_select(0, indices)


def _scatter_rows(values, indices, total):
    full = torch.zeros(total, device=values.device, dtype=values.dtype)
    return full.index_copy_(0, indices, values.detach())


def fused_head(hidden, weight, labels, num_items_in_batch=None, *, packed=None):
    """(loss, HeadStep) of the causal-LM cross-entropy without full logits.

    hidden [B, S, H] aligned with labels [B, S], or, with ``packed`` =
    (batch, packed_hidden [1, T, H]), the packed real positions of that batch.
    weight is the head [V, H]; a head that requires grad gets its gradient too.
    """
    from .kernels.cross_entropy import fused_linear_cross_entropy

    if packed is not None:
        batch, packed_hidden = packed
        rows = packed_hidden.reshape(-1, packed_hidden.shape[-1])
        head_targets = select_targets(labels, batch.indices)
    else:
        rows = hidden.reshape(-1, hidden.shape[-1])
        head_targets = select_targets(labels)
    token_loss, entropy, argmax, _ = fused_linear_cross_entropy(
        rows.contiguous(), weight, head_targets, IGNORE, weight_grad=weight.requires_grad)
    labelled_mask = head_targets != IGNORE
    denominator = labelled_mask.sum() if num_items_in_batch is None else num_items_in_batch
    if isinstance(denominator, torch.Tensor):
        denominator = denominator.to(token_loss.device)
    loss = token_loss.sum() / denominator
    with torch.no_grad():
        correct = ((argmax == head_targets) & labelled_mask).sum()
        labelled = labelled_mask.sum()
        if packed is not None:
            token_loss_full = _scatter_rows(token_loss, batch.indices, labels.numel())
            entropy_full = _scatter_rows(entropy, batch.indices, labels.numel())
        else:
            token_loss_full, entropy_full = token_loss.detach(), entropy.detach()
        step = HeadStep(token_loss=token_loss_full.reshape(labels.shape),
                        token_entropy=entropy_full.reshape(labels.shape),
                        correct=correct, labelled=labelled)
    return loss, step


def _head_weight_ok(head, hidden):
    w = getattr(head, "weight", None)
    return (type(head) is torch.nn.Linear and head.bias is None
            and not (head._forward_hooks or head._forward_pre_hooks)
            and isinstance(w, torch.Tensor) and w.is_cuda and w.device == hidden.device
            and w.dtype in (torch.float16, torch.float32) and w.ndim == 2
            and w.shape[1] == hidden.shape[-1]
            and (hidden.dtype == w.dtype or torch.is_autocast_enabled("cuda")))


def _call_ok(labels, logits_to_keep, kwargs):
    return (enabled() and isinstance(labels, torch.Tensor) and labels.is_cuda
            and labels.dtype == torch.int64 and labels.ndim == 2
            and isinstance(logits_to_keep, int) and logits_to_keep == 0
            and kwargs.get("return_dict", True) is not False
            and not kwargs.get("output_attentions") and not kwargs.get("output_hidden_states"))


def build_causal_lm_forward(original, module):
    cls = getattr(module, "Qwen2ForCausalLM", None)
    if not isinstance(cls, type) or cls.__module__ != module.__name__:
        return None

    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, labels=None, use_cache=None,
                logits_to_keep=0, **kwargs):
        model_args = dict(input_ids=input_ids, attention_mask=attention_mask,
                          position_ids=position_ids, past_key_values=past_key_values,
                          inputs_embeds=inputs_embeds, use_cache=use_cache, **kwargs)
        from .norm_scope import final_norm_half_ready, half_norm_scope

        exact = type(self) is cls
        owner = self.model.norm if exact and final_norm_half_ready(self, kwargs) else None
        if not exact or not _call_ok(labels, logits_to_keep, kwargs):
            with half_norm_scope(owner):
                return original(self, labels=labels, logits_to_keep=logits_to_keep, **model_args)
        num_items = kwargs.pop("num_items_in_batch", None)
        model_args.pop("num_items_in_batch", None)
        from .unpad_route import HEAD_LABELS, take_packed_head

        token = HEAD_LABELS.set((labels, attention_mask))
        try:
            with half_norm_scope(owner):
                outputs = self.model(**model_args)
        finally:
            HEAD_LABELS.reset(token)
        hidden = outputs.last_hidden_state
        packed = take_packed_head(self.model, hidden)
        if (isinstance(hidden, torch.Tensor) and hidden.shape[:2] == labels.shape
                and hidden.dtype in (torch.float16, torch.float32)
                and _head_weight_ok(self.lm_head, hidden)):
            loss, step = fused_head(hidden, self.lm_head.weight, labels, num_items, packed=packed)
            self._soupsuck_head_step = step
            logits = None
        else:
            logits = self.lm_head(hidden)
            loss = self.loss_function(logits=logits, labels=labels,
                                      vocab_size=self.config.vocab_size,
                                      num_items_in_batch=num_items, **kwargs)
        from transformers.modeling_outputs import CausalLMOutputWithPast

        return CausalLMOutputWithPast(loss=loss, logits=logits,
                                      past_key_values=outputs.past_key_values,
                                      hidden_states=outputs.hidden_states,
                                      attentions=outputs.attentions)

    return forward
