"""Casts of expert weights kept between calls while the weights are unchanged.

An expert weight is cast to MXFP8 twice per use: along K for the forward GEMM
and along N for the data gradient (quant_weight_dual does both from one read).
Weights change only at the optimizer step, so calls between two steps
(gradient-accumulation micro-batches, forward-only evaluation, activation
recomputation) can share one pair of casts.  The reference re-quantises its
weights on every call (e2e_bench.py:35-40, memory/2026-06-09.md:25 names the
prepack cache as the next step); this cache is the library's answer.

A cached entry is used only while it is provably current: same tensor object
(held weakly), same storage pointer, shape, strides and in-place version
counter (every in-place update, including optimizer steps, bumps it).  Writes
through `.data` or from outside torch do not bump the version counter, so
caching is opt-in: pass a cache to the ops that accept one.
"""
from __future__ import annotations

import weakref
from collections import OrderedDict

import torch

from . import ops


class WeightCastCache:
    """LRU cache of quant_weight_dual results keyed on the weight's identity and
    version.  `max_entries` bounds the number of weights held (each entry is
    about two e4m3 copies of the weight plus scales)."""

    def __init__(self, max_entries: int = 16, cast=None):
        self.max_entries = max_entries
        self._cast = cast or ops.quant_weight_dual
        self._entries: OrderedDict = OrderedDict()
        self.hits = 0
        self.misses = 0

    @staticmethod
    def _key(w: torch.Tensor, scaling_mode: str):
        return (id(w), w.data_ptr(), w._version, tuple(w.shape), tuple(w.stride()), str(w.device),
                str(scaling_mode))

    def get(self, w: torch.Tensor, scaling_mode: str = "rceil"):
        """((wq, ws), (wt, wts)) for w, from the cache when w is unchanged."""
        key = self._key(w, scaling_mode)
        entry = self._entries.get(key)
        if entry is not None and entry[0]() is w:
            self._entries.move_to_end(key)
            self.hits += 1
            return entry[1]
        self.misses += 1
        value = self._cast(w, scaling_mode)
        # drop stale entries of the same tensor (older versions)
        for k in [k for k in self._entries if k[0] == key[0]]:
            del self._entries[k]
        self._entries[key] = (weakref.ref(w), value)
        while len(self._entries) > self.max_entries:
            self._entries.popitem(last=False)
        return value

    def clear(self) -> None:
        self._entries.clear()

    def __len__(self) -> int:
        return len(self._entries)
