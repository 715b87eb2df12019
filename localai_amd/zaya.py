"""GPU drop-in for ZAYA's MoE block: `ZayaModel._moe(layer, h, prev_router)`
(engine/zaya.py:274-307), the router MLP and the top-1 expert FFN (or the
learned skip route) on the device.

    class ZayaModel(ZayaMoEMixin, LlamaModel): ...   # _moe and _expert_matvec now run on the GPU

Per MoE layer:
  r0      = W_inp h (+ bias)          matvec kernels on the device copy of
                                      blk.L.ffn_gate_inp.weight
  router  tail (one launch)           EDA, RMSNorm, two GELU projections, the
                                      logits, softmax, + learned biases, argmax
                                      (localai_hip_zaya_router)
  expert e < E                        gate_up[e] h, SiLU * up, down[e] act,
                                      times probs[e] (engine/zaya.py:303-306)
  e == E (skip)                       h * probs[E] (:297-301)
Q4_K / Q6_K / Q8_0 experts run as one launch that reads the chosen index and its
probability on the device (localai_hip_moe_experts1, the skip route
included), so the host waits only for the outputs. Other expert types take
the matvec path: the host reads the index (four bytes) to pick the expert
tensors, as the reference's Python does. Returns (moe [dim] float32,
router_state [R] float32) like the reference.

Tensors come from `self.gguf`: a localai_amd.gguf.GGUFFile keeps the device
copies with the file; any other reader with `.tensors` and `._map` (the
reference's GGUFFile) gets copies cached on the model. The router's small
matrices are decoded once to fp32 on the device.

Rounding: the router follows the reference's fp32 steps (see
csrc/zaya.hip); the matvec and softmax sums and the exponential are not
bit-identical to NumPy's, so an expert choice can differ from the
reference's only when two routes are within a few fp32 ulps.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, device
from .dequant import block_layout, dequantize_device
from .moe import ZayaExpertsMixin


class _Layer:
    pass


class ZayaMoEMixin(ZayaExpertsMixin):
    """`_moe(layer, h, prev_router)` with the signature and semantics of
    engine/zaya.py:274-307. Needs `self.gguf`, `self.n_experts`, `self.eps`."""

    # ---- device copies --------------------------------------------------

    def _zaya_cache(self):
        c = getattr(self, '_zaya_dev', None)
        if c is None:
            c = self._zaya_dev = {}
        return c

    def _zaya_raw(self, name):
        g = self.gguf
        if hasattr(g, 'raw_tensor'):
            return g.raw_tensor(name)
        info = g.tensors[name]
        block, bpb = block_layout(info.ggml_type)
        n = int(np.prod(info.shape, dtype=np.int64))
        return memoryview(g._map)[info.offset:info.offset + n // block * bpb]

    def _zaya_f32(self, name):
        """fp32 device copy of tensor `name` (any GGML type), shape as in the file."""
        cache = self._zaya_cache()
        key = ('f32', name)
        if key not in cache:
            info = self.gguf.tensors[name]
            raw = self._zaya_raw(name)
            try:
                cache[key] = dequantize_device(raw, info.ggml_type, info.shape)
            finally:
                if isinstance(raw, memoryview):
                    raw.release()
        return cache[key]

    def _zaya_matrix(self, name):
        """Device matrix (QMat or fp32 DenseMatrix) with .matvec(x, expert=)."""
        dm = getattr(self.gguf, 'device_matrix', None)
        if dm is not None:
            return dm(name)
        cache = self._zaya_cache()
        key = ('mat', name)
        if key not in cache:
            from .gguf import _PACKED, DenseMatrix
            info = self.gguf.tensors[name]
            batch = info.shape[0] if len(info.shape) == 3 else 1
            rows, cols = info.shape[-2], info.shape[-1]
            raw = self._zaya_raw(name)
            try:
                if info.ggml_type in _PACKED:
                    m = device.QMat.from_ggml(raw, info.ggml_type, rows, cols, batch)
                else:
                    m = DenseMatrix(dequantize_device(raw, info.ggml_type, (batch * rows, cols)), batch, rows, cols)
            finally:
                if isinstance(raw, memoryview):
                    raw.release()
            cache[key] = m
        return cache[key]

    def _zaya_bias(self, name):
        b = name[:-6] + 'bias' if name.endswith('.weight') else ''
        return self._zaya_f32(b) if b and b in self.gguf.tensors else None

    def _zaya_layer(self, layer):
        cache = self._zaya_cache()
        key = ('layer', layer)
        if key in cache:
            return cache[key]
        p = f'blk.{layer}.'
        L = _Layer()
        L.inp = p + 'ffn_gate_inp.weight'
        L.b_inp = self._zaya_bias(L.inp)
        eda = p + 'zaya_router_eda.weight'
        L.eda = self._zaya_f32(eda) if eda in self.gguf.tensors else None
        L.norm = self._zaya_f32(p + 'ffn_norm.weight')
        L.w1 = self._zaya_f32(p + 'ffn_gate.weight')
        L.b1 = self._zaya_bias(p + 'ffn_gate.weight')
        L.w2 = self._zaya_f32(p + 'zaya_router_mlp2.weight')
        L.b2 = self._zaya_bias(p + 'zaya_router_mlp2.weight')
        L.w3 = self._zaya_f32(p + 'zaya_router_mlp4.weight')
        L.b3 = self._zaya_bias(p + 'zaya_router_mlp4.weight')
        L.route_bias = self._zaya_f32(p + 'zaya_router_biases.weight')
        L.R = int(self.gguf.tensors[L.inp].shape[0])
        L.R1, L.R2 = int(L.w1.shape[0]), int(L.w2.shape[0])
        L.routes = int(L.w3.shape[0])
        if (tuple(L.w1.shape) != (L.R1, L.R) or tuple(L.w2.shape) != (L.R2, L.R1)
                or tuple(L.w3.shape) != (L.routes, L.R2) or L.routes != self.n_experts + 1
                or L.route_bias.numel() != L.routes or L.norm.numel() != L.R):
            raise ValueError(f'{p}: router tensors do not chain ({L.R} -> {L.R1} -> {L.R2} -> {L.routes})')
        cache[key] = L
        return L

    # ---- the block ----------------------------------------------------------

    def _zaya_experts1(self, p, h_d, expert, expert_w, out, s):
        """The expert FFN (or the skip route) in one launch from the device-side
        choice; False when the experts' type has no such kernel."""
        cache = self._zaya_cache()
        if cache.get(('experts1', p)) is False:
            return False
        gu = self._zaya_matrix(p + 'ffn_gate_up_exps.weight')
        dn = self._zaya_matrix(p + 'ffn_down_exps.weight')
        if not (isinstance(gu, device.QMat) and isinstance(dn, device.QMat)):
            cache[('experts1', p)] = False
            return False
        t = device.torch()
        lib = _lib.load()
        H, I = h_d.numel(), gu.rows // 2
        key = ('experts1_ws', gu.batch, H, I)
        if key not in cache:
            n = int(lib.localai_hip_moe_workspace_size(1, gu.batch, 1, H, I))
            if n < 0:
                raise ValueError(f'{p}: no MoE workspace for experts={gu.batch} hidden={H} inter={I}')
            cache[key] = t.empty(n, dtype=t.uint8, device=h_d.device)
        ws = cache[key]
        ptr = device.ptr
        st = lib.localai_hip_moe_experts1(ptr(h_d), H, gu.handle, dn.handle, 1, ptr(expert), ptr(expert_w),
                                          self.n_experts, ptr(out), ptr(ws), ws.numel(), s)
        if st == 2:   # ETYPE: not Q4_K / Q6_K / Q8_0 on the tile form
            cache[('experts1', p)] = False
            return False
        _lib.check(st)
        return True

    def _moe(self, layer, h, prev_router):
        t = device.torch()
        lib = _lib.load()
        L = self._zaya_layer(layer)
        p = f'blk.{layer}.'
        hv = np.asarray(h, dtype=np.float32).reshape(-1)
        h_d = device.to_device_f32(hv)
        r0 = self._zaya_matrix(L.inp).matvec(h_d).reshape(-1)
        prev_d = None
        if L.eda is not None and prev_router is not None:
            prev_d = device.to_device_f32(np.asarray(prev_router, dtype=np.float32).reshape(-1))
            if prev_d.numel() != L.R:
                raise ValueError(f'prev_router has {prev_d.numel()} values, the router state has {L.R}')
        dev = h_d.device
        state = t.empty(L.R, dtype=t.float32, device=dev)
        probs = t.empty(L.routes, dtype=t.float32, device=dev)
        expert = t.empty(1, dtype=t.int32, device=dev)
        expert_w = t.empty(1, dtype=t.float32, device=dev)
        ptr = device.ptr
        opt = lambda v: ptr(v) if v is not None else None   # noqa: E731
        s = ctypes.c_void_p(device.stream_ptr())
        _lib.check(lib.localai_hip_zaya_router(
            ptr(r0), opt(L.b_inp), opt(prev_d), opt(L.eda if prev_d is not None else None), ptr(L.norm),
            ctypes.c_float(self.eps), L.R, ptr(L.w1), opt(L.b1), L.R1, ptr(L.w2), opt(L.b2), L.R2, ptr(L.w3),
            opt(L.b3), L.routes, ptr(L.route_bias), ptr(state), ptr(probs), ptr(expert), ptr(expert_w), s))
        out = t.empty(hv.size, dtype=t.float32, device=dev)
        if self._zaya_experts1(p, h_d, expert, expert_w, out, s):
            ws = self._zaya_cache()[('experts1_ws', self.n_experts, hv.size,
                                     self._zaya_matrix(p + 'ffn_gate_up_exps.weight').rows // 2)]
            _lib.check(lib.localai_hip_moe_error(ptr(ws), 1, self.n_experts, s))   # waits for the stream
            return out.cpu().numpy(), state.cpu().numpy()
        e = int(expert.cpu().item())
        scale = probs[e:e + 1]
        if e == self.n_experts:
            _lib.check(lib.localai_hip_zaya_scale(None, ptr(h_d), hv.size, ptr(scale), ptr(out), s))
        else:
            gu = self._zaya_matrix(p + 'ffn_gate_up_exps.weight').matvec(h_d, expert=e).reshape(-1)
            inter = gu.numel() // 2
            act = t.empty(inter, dtype=t.float32, device=dev)
            _lib.check(lib.localai_hip_zaya_scale(ptr(gu), None, inter, None, ptr(act), s))
            y = self._zaya_matrix(p + 'ffn_down_exps.weight').matvec(act, expert=e).reshape(-1)
            _lib.check(lib.localai_hip_zaya_scale(None, ptr(y), hv.size, ptr(scale), ptr(out), s))
        return out.cpu().numpy(), state.cpu().numpy()
