"""Top-k MoE expert layer on the GPU, and the ZAYA expert-matvec drop-in.

MoELayer        device-resident router + quantized expert tensors; forward()
                runs route -> permute -> grouped gate_up (+SiLU*up) -> grouped
                down -> weighted combine (liblocalai_hip.so, one stream).
expert_matvec   W[e] @ x for expert e of a [E, rows, cols] GGML tensor; the
                semantics of ZayaModel._expert_matvec (engine/zaya.py:139-175):
                expert e is the byte slice [e*B, (e+1)*B) of the tensor.
ZayaExpertsMixin
                provides `_expert_matvec(self, name, expert, x)` with the
                reference signature for a model holding `self.gguf`: a
                localai_amd.gguf.GGUFFile (the expert tensor's device copy
                lives with the file), or any reader with `.tensors[name]` ->
                (shape, ggml_type, offset) and `._map`.

Selection semantics (generalising engine/zaya.py:290-306 to top-k): router
logits are ranked (value desc, index asc: the np.argmax tie rule of
engine/zaya.py:296); gates are the softmax over the k selected logits; expert
output = W_down[e] @ (silu(g) * u) with [g; u] = W_gate_up[e] @ h (first half
gate, engine/zaya.py:303-305).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, device
from .dequant import block_layout


class MoELayer:
    def __init__(self, router_w, gate_up_raw, down_raw, ggml_type, n_experts, hidden, inter, top_k,
                 router_b=None, down_type=None):
        t = device.torch()
        self.E, self.H, self.I, self.k = int(n_experts), int(hidden), int(inter), int(top_k)
        dev = device.device()
        rw = np.ascontiguousarray(router_w, dtype=np.float32)
        if rw.shape != (self.E, self.H):
            raise ValueError(f'router weight must be [{self.E}, {self.H}], got {rw.shape}')
        self.router_w = t.from_numpy(rw.copy()).to(dev)
        self.router_b = None
        if router_b is not None:
            self.router_b = t.from_numpy(np.ascontiguousarray(router_b, dtype=np.float32).copy()).to(dev)
        self.gate_up = device.QMat.from_ggml(gate_up_raw, ggml_type, 2 * self.I, self.H, self.E)
        self.down = device.QMat.from_ggml(down_raw, down_type or ggml_type, self.H, self.I, self.E)
        self._ws = {}

    def workspace(self, tokens):
        ws = self._ws.get(tokens)
        if ws is None:
            n = int(_lib.load().localai_hip_moe_workspace_size(tokens, self.E, self.k, self.H, self.I))
            if n < 0:
                raise ValueError('invalid MoE sizes')
            ws = device.torch().empty(n, dtype=device.torch().uint8, device=device.device())
            self._ws[tokens] = ws
        return ws

    def forward_device(self, h, out=None, idx=None, gates=None, stream=None):
        """h: [T, H] fp32 device tensor -> (out [T, H], topk_idx [T, k] int32, gates [T, k])."""
        t = device.torch()
        if h.dim() == 1:
            h = h.reshape(1, -1)
        if h.dtype != t.float32 or not h.is_contiguous() or h.data_ptr() % 16:
            h = h.to(t.float32).contiguous().clone()
        T = h.shape[0]
        if h.shape[1] != self.H:
            raise ValueError(f'h has {h.shape[1]} features, layer expects {self.H}')
        dev = h.device
        out = out if out is not None else t.empty((T, self.H), dtype=t.float32, device=dev)
        idx = idx if idx is not None else t.empty((T, self.k), dtype=t.int32, device=dev)
        gates = gates if gates is not None else t.empty((T, self.k), dtype=t.float32, device=dev)
        ws = self.workspace(T)
        rb = device.ptr(self.router_b) if self.router_b is not None else None
        _lib.check(_lib.load().localai_hip_moe_forward(
            device.ptr(h), T, self.H, device.ptr(self.router_w), rb, self.E, self.k,
            self.gate_up.handle, self.down.handle, device.ptr(out), device.ptr(idx), device.ptr(gates),
            device.ptr(ws), ws.numel(), ctypes.c_void_p(device.stream_ptr(stream))))
        return out, idx, gates

    def last_router_logits(self, tokens):
        """Router logits [tokens, E] (fp32, bias included) of the last forward
        over `tokens` tokens: the layer's workspace starts with them."""
        ws = self._ws.get(tokens)
        if ws is None:
            raise ValueError(f'no forward over {tokens} tokens yet')
        return ws[:tokens * self.E * 4].view(device.torch().float32).reshape(tokens, self.E)

    def last_tables(self, tokens):
        """Routing tables of the last forward over `tokens` tokens, as numpy
        int32 arrays: counts, offsets, active (n_active of them), perm, pos and,
        from 32 tokens on, the expert GEMM tiles (tile_e, tile_p0, tile_n) and
        their width tile_w."""
        ws = self._ws.get(tokens)
        if ws is None:
            raise ValueError(f'no forward over {tokens} tokens yet')
        offs = (ctypes.c_int64 * 12)()
        _lib.check(_lib.load().localai_hip_moe_table_offsets(tokens, self.E, self.k, self.H, self.I, offs))
        host = ws.cpu().numpy()
        E, N = self.E, tokens * self.k

        def ints(i, n):
            return host[offs[i]:offs[i] + 4 * n].view(np.int32).copy()

        t = {'counts': ints(0, E), 'offsets': ints(1, E + 1), 'perm': ints(4, N), 'pos': ints(5, N)}
        t['active'] = ints(2, int(ints(3, 1)[0]))
        if offs[9] >= 0:
            nt = int(ints(9, 1)[0])
            t['tile_e'], t['tile_p0'], t['tile_n'] = ints(6, nt), ints(7, nt), ints(8, nt)
            t['tile_w'] = int(offs[11])
        return t

    def check(self, tokens, stream=None):
        """Wait for `stream` and raise if the last forward over `tokens` tokens
        ran the fused one-token expert kernel and one of its device-side checks
        failed (an expert index out of range, or a hand-off wait that ran out:
        its output rows are then NaN)."""
        ws = self._ws.get(tokens)
        if ws is not None:
            _lib.check(_lib.load().localai_hip_moe_error(device.ptr(ws), tokens, self.E,
                                                          ctypes.c_void_p(device.stream_ptr(stream))))

    def forward(self, h):
        """numpy [T, H] -> numpy (out [T, H], topk_idx [T, k], gates [T, k])."""
        h = np.atleast_2d(h)
        o, i, g = self.forward_device(device.to_device_f32(h))
        self.check(h.shape[0])
        return o.cpu().numpy(), i.cpu().numpy(), g.cpu().numpy()


def expert_matvec(tensor_raw, shape, ggml_type, expert, x):
    """W[expert] @ x for a [E, rows, cols] GGML tensor given as host bytes.

    The whole 3-D tensor is uploaded once (in native_quant's weight cache when
    `tensor_raw` is immutable) and expert `expert` is addressed inside it,
    like the byte slicing of engine/zaya.py:144-150.
    """
    from . import native_quant
    E, rows, cols = (int(s) for s in shape)
    block, bpb = block_layout(ggml_type)
    if cols % block:
        raise ValueError('expert dimensions do not align to quant blocks')
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    if x.size != cols:
        raise ValueError(f'expert input has {x.size} values, expected {cols}')
    if not 0 <= int(expert) < E:
        raise IndexError(f'expert {expert} outside [0, {E})')
    _, nbytes = device.host_address(tensor_raw)
    if nbytes != E * rows * (cols // block) * bpb:
        raise ValueError('tensor bytes do not match [E, rows, cols]')
    q = native_quant.weights(tensor_raw, rows, cols, ggml_type, batch=E)
    return q.matvec(device.to_device_f32(x), expert=int(expert)).cpu().numpy()


class ZayaExpertsMixin:
    """`_expert_matvec(name, expert, x)` with the signature of engine/zaya.py:139."""

    def _expert_matvec(self, name, expert, x):
        info = self.gguf.tensors[name]
        if len(info.shape) != 3 or info.shape[0] != self.n_experts:
            raise ValueError(f'{name}: expected [experts,out,in], got {info.shape}')
        device_matrix = getattr(self.gguf, 'device_matrix', None)
        if device_matrix is not None:
            # localai_amd.gguf.GGUFFile: the tensor's device copy lives with the file
            E, rows, cols = info.shape
            if not 0 <= int(expert) < E:
                raise IndexError(f'expert {expert} outside [0, {E})')
            xv = np.asarray(x, dtype=np.float32).reshape(-1)
            if xv.size != cols:
                raise ValueError(f'expert input has {xv.size} values, expected {cols}')
            q = device_matrix(name)
            return q.matvec(device.to_device_f32(xv), expert=int(expert)).cpu().numpy()
        block, bpb = block_layout(info.ggml_type)
        E, rows, cols = info.shape
        nbytes = E * rows * (cols // block) * bpb
        raw = memoryview(self.gguf._map)[info.offset:info.offset + nbytes]
        return expert_matvec(raw, info.shape, info.ggml_type, expert, x)
