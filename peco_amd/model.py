"""Installing PECO on a transformer (the peco/model.py interface: install_attention, reset_state).

An installation is one object kept on the transformer. It owns the shared
``InferenceContext``, one ``PecoAttention`` per attention block (double-stream blocks first,
then single-stream blocks, so a processor's index is its layer index) and the forward
pre-hook that refreshes the context before every transformer call. Installing again replaces
the previous installation: its hook is removed first, so a transformer never advances the
step twice per call.

Works with any pipeline whose ``transformer`` has ``transformer_blocks`` and
``single_transformer_blocks`` (blocks with ``attn.set_processor``) and a ``forward`` that
takes ``encoder_attention_mask`` (HunyuanVideo in diffusers).
"""
from __future__ import annotations

import inspect
from dataclasses import dataclass, field

import torch

from .processor import InferenceContext, PecoAttention, PecoConfig

_ATTRIBUTE = "_peco_installation"


def _text_lengths(mask):
    """(total, valid) text lengths of one prompt's right-padded mask [1, T].

    The reference's hook accepts exactly one prompt and masks whose valid tokens form a
    prefix (peco/model.py:25-34); the same errors are raised here.
    """
    if mask.shape[0] != 1:
        raise ValueError("Use one prompt per inference call")
    row = mask[0].detach().to(device="cpu", dtype=torch.bool)
    valid = int(row.sum())
    prefix = torch.arange(row.numel()) < valid
    if not torch.equal(row, prefix):
        raise ValueError("Hunyuan text attention mask must use right padding")
    return row.numel(), valid


@dataclass
class _Installation:
    context: InferenceContext
    processors: list
    signature: inspect.Signature
    handle: object = field(default=None)

    def before_forward(self, module, args, kwargs):
        """Forward pre-hook: one transformer call is one denoising step."""
        bound = self.signature.bind_partial(*args, **kwargs).arguments
        total, valid = _text_lengths(bound["encoder_attention_mask"])
        self.context.step += 1
        self.context.text_length = total
        self.context.valid_text_length = valid

    def reset(self):
        self.context.step = -1
        for processor in self.processors:
            processor.reset()

    def remove(self):
        if self.handle is not None:
            self.handle.remove()
            self.handle = None


def install_attention(pipe, config: PecoConfig):
    """Give every attention block of ``pipe.transformer`` a PecoAttention; return the shared context."""
    transformer = pipe.transformer
    old = getattr(transformer, _ATTRIBUTE, None)
    if old is not None:
        old.remove()
    attentions = [block.attn for block in (*transformer.transformer_blocks, *transformer.single_transformer_blocks)]
    context = InferenceContext()
    installation = _Installation(context, [PecoAttention(i, config, context) for i in range(len(attentions))],
                                 inspect.signature(transformer.forward))
    for attn, processor in zip(attentions, installation.processors):
        attn.set_processor(processor)
    installation.handle = transformer.register_forward_pre_hook(installation.before_forward, with_kwargs=True)
    setattr(transformer, _ATTRIBUTE, installation)
    return context


def reset_state(pipe):
    """Forget the step count and every layer's cached centroids (call before each new video)."""
    getattr(pipe.transformer, _ATTRIBUTE).reset()
