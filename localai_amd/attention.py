"""The attention mixers of a decode step on the GPU.

    KVCache           device counterpart of the reference's KVCache
                      (engine/model.py:6-9): k and v [n_layers, max_seq,
                      n_kv_heads, head_dim] fp32, plus the attention workspace
    attention_decode  grouped-query attention of one token over one layer of
                      the cache (engine/model.py:222-227; with `gate`, Qwen3.5's
                      gated full attention, engine/qwen35.py:158-182)
    delta_net_step    the gated delta-rule step of Qwen3.5's linear attention,
                      with the signature of engine/numba_kernels.py:12

Arguments are fp32 device tensors; the work runs in the HIP library
(localai_hip_attention_decode, localai_hip_delta_net_step) and nothing here
computes on the host.
"""
from __future__ import annotations

import ctypes

from . import _lib, device


def _dev_f32(t, name, numel=None):
    torch = device.torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f'{name} must be a device tensor')
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise TypeError(f'{name} must be a contiguous float32 tensor')
    if numel is not None and t.numel() != numel:
        raise ValueError(f'{name} must have {numel} values, got {t.numel()}')
    return t


class KVCache:
    """engine/model.py:6-9 on the device: k, v [n_layers, max_seq, n_kv_heads,
    head_dim] fp32 (zero-filled), `length`, reset()."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq, n_heads=None):
        torch = device.torch()
        dev = device.device()
        self.k = torch.zeros((n_layers, max_seq, n_kv_heads, head_dim), dtype=torch.float32, device=dev)
        self.v = torch.zeros_like(self.k)
        self.length = 0
        self.max_seq = int(max_seq)
        self.n_kv_heads, self.head_dim = int(n_kv_heads), int(head_dim)
        self.n_heads = int(n_heads) if n_heads else self.n_kv_heads
        n = int(_lib.load().localai_hip_attention_workspace_size(self.max_seq, self.n_heads, self.n_kv_heads,
                                                                   self.head_dim))
        if n < 0:
            raise ValueError('invalid attention sizes')
        self.ws = torch.empty(max(n, 256), dtype=torch.uint8, device=dev)

    def reset(self):
        self.length = 0


def attention_decode(q, k, v, cache, layer, position, n_heads, window=0, gate=None, out=None, stream=None):
    """Write k, v ([n_kv_heads * head_dim] each; None: the row is already in
    the cache) at `position` of cache layer `layer` and return the attention
    output [n_heads * head_dim] of query q ([n_heads * head_dim]) over positions
    max(0, position + 1 - window) .. position (all up to `position` for
    window <= 0). gate: Qwen3.5's output gate [n_heads * head_dim] or None."""
    torch = device.torch()
    hd, nkv = cache.head_dim, cache.n_kv_heads
    if n_heads != cache.n_heads:
        raise ValueError(f'the cache was sized for {cache.n_heads} query heads')
    _dev_f32(q, 'q', n_heads * hd)
    if (k is None) != (v is None):
        raise ValueError('k and v go together')
    if k is not None:
        _dev_f32(k, 'k', nkv * hd)
        _dev_f32(v, 'v', nkv * hd)
    if gate is not None:
        _dev_f32(gate, 'gate', n_heads * hd)
    if not 0 <= layer < cache.k.shape[0]:
        raise IndexError('layer out of range')
    if out is None:
        out = torch.empty(n_heads * hd, dtype=torch.float32, device=q.device)
    _dev_f32(out, 'out', n_heads * hd)
    p = device.ptr
    kc, vc = cache.k[layer], cache.v[layer]
    _lib.check(_lib.load().localai_hip_attention_decode(
        p(q), p(k) if k is not None else None, p(v) if v is not None else None, p(kc), p(vc), int(position),
        cache.max_seq, int(n_heads), nkv, hd, int(max(window, 0)), p(gate) if gate is not None else None, p(out),
        p(cache.ws), cache.ws.numel(), ctypes.c_void_p(device.stream_ptr(stream))))
    cache.length = max(cache.length, int(position) + 1)
    return out


def delta_net_step(state, q, k, v, decay, beta, core=None, stream=None):
    """engine/numba_kernels.py:12: state [heads, key_dim, value_dim] is
    updated in place; returns core [heads, value_dim]. q, k [heads, key_dim],
    v [heads, value_dim], decay and beta [heads]: fp32 device tensors."""
    torch = device.torch()
    _dev_f32(state, 'state')
    if state.dim() != 3:
        raise ValueError('state must be [heads, key_dim, value_dim]')
    heads, kd, vd = (int(x) for x in state.shape)
    _dev_f32(q, 'q', heads * kd)
    _dev_f32(k, 'k', heads * kd)
    _dev_f32(v, 'v', heads * vd)
    _dev_f32(decay, 'decay', heads)
    _dev_f32(beta, 'beta', heads)
    if core is None:
        core = torch.empty((heads, vd), dtype=torch.float32, device=state.device)
    _dev_f32(core, 'core', heads * vd)
    p = device.ptr
    _lib.check(_lib.load().localai_hip_delta_net_step(p(state), p(q), p(k), p(v), p(decay), p(beta), p(core),
                                                      heads, kd, vd, ctypes.c_void_p(device.stream_ptr(stream))))
    return core
