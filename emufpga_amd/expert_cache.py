"""Experts in host memory behind HBM slots (emu_expert_cache).

Mirrors spm-granite-moe's ExpertCache (src/expert_cache.rs:20-90: admit on
the second use, least-recently-used eviction under a byte budget) with the
layer-aware victim choice of tools/llama-logits/mmid-cache.hpp:134-173, in
front of the GPU: the budget is a number of HBM slots of one expert each,
the backing store pinned host memory, and ``moe_ffn`` runs the selected-expert
FFN (moe::run, moe.rs:124-159) on whatever the cache holds or streams through.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import ExpertCacheStats, MoeDesc
from .device import Context


def policy_trace(n_slots: int, layer_aware: bool, calls, layers, experts) -> tuple[np.ndarray, np.ndarray]:
    """The cache policy alone (no device): outcome per lookup (0 hit, 1
    admitted, 2 streamed through) and its slot (-1 when streamed)."""
    from ._lib import load
    lib = load()
    n = len(calls)
    arrs = [np.ascontiguousarray(a, np.uint32) for a in (calls, layers, experts)]
    out, slot = np.empty(n, np.int32), np.empty(n, np.int32)
    st = lib.emu_expert_cache_policy_trace(n_slots, int(layer_aware), *[a.ctypes.data_as(C.c_void_p) for a in arrs],
                                           n, out.ctypes.data_as(C.c_void_p), slot.ctypes.data_as(C.c_void_p))
    if st != 0:
        raise ValueError(f"policy trace failed ({st})")
    return out, slot


class ExpertCache:
    """n_slots resident HBM slots and n_transient stream-through slots for
    experts of expert_bytes (gate rows, up rows, down rows back to back)."""

    def __init__(self, ctx: Context, layers: int, n_experts: int, expert_bytes: int, n_slots: int,
                 n_transient: int, layer_aware: bool = False):
        self.ctx, self.layers, self.n_experts, self.expert_bytes = ctx, layers, n_experts, expert_bytes
        h = C.c_void_p()
        ctx.check(ctx.lib.emu_expert_cache_create(ctx.h, layers, n_experts, expert_bytes, n_slots, n_transient,
                                                  int(layer_aware), C.byref(h)), "emu_expert_cache_create")
        self.h = h
        self._host = []

    def set_layer(self, layer: int, experts: np.ndarray) -> None:
        """Copy one layer's experts (n_experts x expert_bytes) into pinned
        host memory and register them as the cache's backing store."""
        experts = np.ascontiguousarray(experts).view(np.uint8).reshape(self.n_experts, self.expert_bytes)
        p = C.c_void_p()
        self.ctx.check(self.ctx.lib.emu_host_alloc(self.ctx.h, experts.size, C.byref(p)), "emu_host_alloc")
        self._host.append(p)
        C.memmove(p, experts.ctypes.data_as(C.c_void_p), experts.size)
        for e in range(self.n_experts):
            self.ctx.check(self.ctx.lib.emu_expert_cache_set_source(self.h, layer, e,
                                                                    C.c_void_p(p.value + e * self.expert_bytes)),
                           "emu_expert_cache_set_source")

    def load_model(self, model) -> None:
        """Every expert of an MoE model (serve.Model) copied from its HBM
        tensors into one pinned host buffer, as the backing store."""
        stride = (self.expert_bytes + 255) // 256 * 256
        nbytes = self.layers * self.n_experts * stride
        p = C.c_void_p()
        self.ctx.check(self.ctx.lib.emu_host_alloc(self.ctx.h, nbytes, C.byref(p)), "emu_host_alloc")
        self._host.append(p)
        self.ctx.check(self.ctx.lib.emu_expert_cache_load_model(self.h, model.h, p, nbytes),
                       "emu_expert_cache_load_model")

    def moe_ffn(self, desc: MoeDesc, layer: int, d_x, n_tok: int, ids: np.ndarray, d_ids, d_weights, d_ws, ws_bytes,
                d_out) -> None:
        ids = np.ascontiguousarray(ids, np.int32)
        self.ctx.check(self.ctx.lib.emu_moe_ffn_cached(self.ctx.h, C.byref(desc), self.h, layer, d_x, n_tok,
                                                       ids.ctypes.data_as(C.c_void_p), d_ids, d_weights, d_ws,
                                                       ws_bytes, d_out), "emu_moe_ffn_cached")

    def stats(self) -> dict:
        s = ExpertCacheStats()
        self.ctx.check(self.ctx.lib.emu_expert_cache_stats(self.h, C.byref(s)), "emu_expert_cache_stats")
        return {f: getattr(s, f) for f, _ in s._fields_}

    def slot(self, layer: int, expert: int) -> int:
        v = C.c_int32()
        self.ctx.check(self.ctx.lib.emu_expert_cache_slot(self.h, layer, expert, C.byref(v)), "emu_expert_cache_slot")
        return v.value

    def close(self) -> None:
        if self.h is not None and self.ctx.live:
            self.ctx.lib.emu_expert_cache_destroy(self.h)
            for p in self._host:
                self.ctx.lib.emu_host_free(self.ctx.h, p)
        self.h = None
        self._host = []


__all__ = ["ExpertCache", "policy_trace"]
