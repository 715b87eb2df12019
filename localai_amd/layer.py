"""The matvec chain of one decode layer (localai_hip_layer_chain).

DecodeLayerChain holds the seven weight handles of the chain -- attn_output,
ffn_gate, ffn_up, ffn_down of layer L and attn_q, attn_k, attn_v of layer
L+1 -- and the two norm weights, and runs, from the attention output of layer
L, the part of the reference's decode step up to the attention inputs of
layer L+1 (engine/model.py:229-233, then :181-185 and :203-210):

    x1 = pre + W_o att;  u = norm(x1) * w_ffn;  act = silu(W_gate u) * (W_up u)
    x_out = x1 + W_down act;  v' = norm(x_out) * w_attn
    q, k, v = W_q v', W_k v', W_v v'   (+ adjacent-pair RoPE of q and k)

All of it stays on the device; nothing here computes on the host. By default
the chain runs as four launches with the glue fused into the matvec kernels;
set_mode(one_launch=True) selects the single launch with device-side waits
between its stages.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, device

ORDER = ('attn_output', 'ffn_gate', 'ffn_up', 'ffn_down', 'attn_q', 'attn_k', 'attn_v')


def set_mode(one_launch):
    """Process-wide: how every DecodeLayerChain runs (False: four launches)."""
    _lib.check(_lib.load().localai_hip_layer_chain_mode(1 if one_launch else 0))


class DecodeLayerChain:
    def __init__(self, mats, w_ffn, w_attn, eps, head_dim=None):
        """mats: name -> device.QMat for the names in ORDER (Q4_K / Q6_K);
        w_ffn: ffn_norm of layer L, w_attn: attn_norm of layer L+1 ([dim] each)."""
        t = device.torch()
        self.mats = [mats[n] for n in ORDER]
        self.dim, self.ffn = self.mats[0].rows, self.mats[1].rows
        self.eps = float(eps)
        self.head_dim = int(head_dim) if head_dim else 0
        dev = device.device()
        self.w_ffn = device.to_device_f32(np.asarray(w_ffn, np.float32).reshape(-1))
        self.w_attn = device.to_device_f32(np.asarray(w_attn, np.float32).reshape(-1))
        if self.w_ffn.numel() != self.dim or self.w_attn.numel() != self.dim:
            raise ValueError(f'norm weights must have {self.dim} values')
        lib = _lib.load()
        n = int(lib.localai_hip_layer_workspace_size(self.dim, self.ffn))
        if n < 0:
            raise ValueError('invalid layer sizes')
        self.ws = t.zeros(n, dtype=t.uint8, device=dev)      # zero-filled once; every launch leaves it so
        self._handles = (ctypes.c_void_p * 7)(*[m.handle.value for m in self.mats])

    def forward_device(self, pre, att, rope=None, out=None, stream=None):
        """pre, att: [dim] fp32 device tensors; rope: (cos, sin) [rope_half]
        fp32 device tensors or None. Returns (x_out [dim], q, k, v)."""
        t = device.torch()
        dev = pre.device
        if out is None:
            out = (t.empty(self.dim, dtype=t.float32, device=dev),
                   t.empty(self.mats[4].rows, dtype=t.float32, device=dev),
                   t.empty(self.mats[5].rows, dtype=t.float32, device=dev),
                   t.empty(self.mats[6].rows, dtype=t.float32, device=dev))
        x_out, q, k, v = out
        p = device.ptr
        cos, sin = rope if rope is not None else (None, None)
        if rope is not None and not self.head_dim:
            raise ValueError('RoPE needs head_dim')
        _lib.check(_lib.load().localai_hip_layer_chain(
            self._handles, p(pre), p(att), p(self.w_ffn), p(self.w_attn), ctypes.c_float(self.eps),
            p(cos) if cos is not None else None, p(sin) if sin is not None else None, self.head_dim,
            int(cos.numel()) if cos is not None else 0, p(x_out), p(q), p(k), p(v), p(self.ws), self.ws.numel(),
            ctypes.c_void_p(device.stream_ptr(stream))))
        return x_out, q, k, v

    def check(self, stream=None):
        """Wait for `stream`; raise if a wait between stages ran out."""
        _lib.check(_lib.load().localai_hip_layer_error(device.ptr(self.ws),
                                                       ctypes.c_void_p(device.stream_ptr(stream))))
