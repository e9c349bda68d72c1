"""MathBrain's Per-Slot EMA hot path on one MI355X (gfx950).

The package keeps the reference's module paths and names, so that its model.py and
train.py imports (``from .triton_flash_ema import FlashEMAFunction``, ``from
mathbrain.model import SlotTransformerLM``, ...) resolve unchanged; the work runs in the
hand-written HIP kernels of ``libmathbrain_hip.so`` (csrc/), loaded on first use.  The
``triton_*`` module names are the reference's import paths: nothing here uses Triton.

File:line citations in this package (``triton_flash_ema.py:571-650``, ``model.py:144``)
name the reference repository's files, not the modules of the same name here.
"""
from .model import SlotTransformerLM
from .baseline import RoPETransformerLM
from .data import WikiTextMMapDataset, preprocess_corpus, dynamic_collate_fn, TokenBudgetSampler

__all__ = ["SlotTransformerLM", "RoPETransformerLM", "WikiTextMMapDataset", "preprocess_corpus",
           "dynamic_collate_fn", "TokenBudgetSampler"]
