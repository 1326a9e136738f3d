"""The head after the encoder on the GPU: the final model's `KneeBaseline` context and per-finding
attention pooling over the HIP library (`d8s_head`, include/d8s_hip.h).

`KneeHead(state_dict)(encoded, slot_of_window, slot_mask)` is `KneeBaseline.forward(None,
slot_of_window, slot_mask, encoded=encoded)` of src/knee/models/baseline.py:1083-1170 for the final
configuration (configs/exp/376-full-data-v9j-287-img512.yaml: attention pooling, one context layer
of width 256 with 4 heads, no slot prior, no window_index): (B, W, D) window features -> (B, 12)
logits, in float32.  The weights are read from the reference's state_dict keys.  There is no CPU path:
without the library the call raises.
"""
from __future__ import annotations

import ctypes

import torch

from . import hip

# reference state_dict key of every D8sHeadArgs weight (src/knee/models/baseline.py:644-713)
KEYS = {
    "slot_emb": "slot_emb", "ctx_in_w": "ctx_in.weight", "ctx_in_b": "ctx_in.bias", "ctx_pos": "ctx_pos",
    "in_proj_w": "ctx.layers.0.self_attn.in_proj_weight", "in_proj_b": "ctx.layers.0.self_attn.in_proj_bias",
    "out_proj_w": "ctx.layers.0.self_attn.out_proj.weight", "out_proj_b": "ctx.layers.0.self_attn.out_proj.bias",
    "ln1_w": "ctx.layers.0.norm1.weight", "ln1_b": "ctx.layers.0.norm1.bias",
    "ln2_w": "ctx.layers.0.norm2.weight", "ln2_b": "ctx.layers.0.norm2.bias",
    "ff1_w": "ctx.layers.0.linear1.weight", "ff1_b": "ctx.layers.0.linear1.bias",
    "ff2_w": "ctx.layers.0.linear2.weight", "ff2_b": "ctx.layers.0.linear2.bias",
    "ctx_out_w": "ctx_out.weight", "ctx_out_b": "ctx_out.bias",
    "attn_w": "attn.weight", "attn_b": "attn.bias", "cls_w": "cls_w", "cls_b": "cls_b",
}


class KneeHead:
    def __init__(self, state_dict: dict, device, context_heads: int = 4) -> None:
        self.device = torch.device(device)
        missing = [k for k in KEYS.values() if k not in state_dict]
        if missing:
            raise KeyError(f"state_dict lacks {missing[:4]} (one context layer and attention pooling "
                           "are required)")
        if "ctx.layers.1.norm1.weight" in state_dict:
            raise ValueError("more than one context layer is not supported")
        self.w = {n: state_dict[k].detach().to(self.device, torch.float32).contiguous()
                  for n, k in KEYS.items()}
        self.S, self.D = self.w["slot_emb"].shape
        self.CD = self.w["ctx_in_w"].shape[0]
        self.PER = self.w["ctx_pos"].shape[0]
        self.FF = self.w["ff1_w"].shape[0]
        self.T = self.w["cls_w"].shape[0]
        self.heads = int(context_heads)
        if self.CD != 64 * self.heads:
            raise ValueError(f"context width {self.CD} with {self.heads} heads: 64 per head is required")
        self._ws: torch.Tensor | None = None
        # the last slot_of_window seen (kept alive, so identity and version name its contents) and
        # its checked int32 copy on the device: a fixed window layout is validated once, not per call
        self._slot_src: torch.Tensor | None = None
        self._slot_ver = -1
        self._slot_dev: torch.Tensor | None = None

    def _args(self, z, slot_of, mask, logits) -> hip.HeadArgs:
        a = hip.HeadArgs()
        a.z, a.slot_of, a.slot_mask, a.logits = z.data_ptr(), slot_of.data_ptr(), mask.data_ptr(), logits.data_ptr()
        for n in hip.HEAD_WEIGHTS:
            setattr(a, n, self.w[n].data_ptr())
        a.B, a.W = z.shape[0], z.shape[1]
        a.D, a.S, a.CD, a.heads, a.FF, a.PER, a.T = self.D, self.S, self.CD, self.heads, self.FF, self.PER, self.T
        a.ctx_layers = 1
        return a

    def _slots(self, slot_of_window: torch.Tensor) -> torch.Tensor:
        """slot_of_window as int32 on the device, checked to lie in 0 .. S-1 (the reference's embedding
        lookup raises on such an index).  The check reads the values on the host, so it runs once per
        tensor and in-place version: later calls with the same unchanged tensor reuse the checked copy."""
        if (self._slot_src is slot_of_window and slot_of_window._version == self._slot_ver
                and self._slot_dev is not None):
            return self._slot_dev
        host = slot_of_window.detach().to("cpu", torch.int64).reshape(-1)
        if bool(((host < 0) | (host >= self.S)).any()):
            raise ValueError("slot_of_window outside 0 .. S-1")
        self._slot_dev = host.to(torch.int32).to(self.device)
        self._slot_src, self._slot_ver = slot_of_window, slot_of_window._version
        return self._slot_dev

    def __call__(self, encoded: torch.Tensor, slot_of_window: torch.Tensor, slot_mask: torch.Tensor,
                 window_index: torch.Tensor | None = None) -> torch.Tensor:
        """encoded (B, W, D), slot_of_window (W,), slot_mask (B, S) bool -> logits (B, T) float32.
        `window_index` is accepted for the reference's signature; this configuration does not use it."""
        if encoded.dim() != 3 or encoded.shape[2] != self.D:
            raise ValueError(f"encoded must be (B, W, {self.D})")
        z = encoded.to(self.device, torch.float32).contiguous()
        slot_of = self._slots(slot_of_window)
        mask = slot_mask.to(self.device)
        mask = mask.view(torch.uint8) if mask.dtype == torch.bool else mask.to(torch.uint8)
        mask = mask.contiguous()
        if slot_of.numel() != z.shape[1] or mask.shape != (z.shape[0], self.S):
            raise ValueError("slot_of_window must have W entries and slot_mask (B, S)")
        logits = torch.empty((z.shape[0], self.T), dtype=torch.float32, device=self.device)
        a = self._args(z, slot_of, mask, logits)
        need = ctypes.c_uint64()
        hip.call("d8s_head_workspace", ctypes.byref(a), ctypes.byref(need))
        if self._ws is None or self._ws.numel() < need.value + 256:
            self._ws = torch.empty(int(need.value) + 256, dtype=torch.uint8, device=self.device)
        base = (self._ws.data_ptr() + 255) // 256 * 256
        a.workspace, a.ws_bytes = base, self._ws.numel() - (base - self._ws.data_ptr())
        stream = torch.cuda.current_stream(self.device).cuda_stream
        hip.call("d8s_head", ctypes.byref(a), ctypes.c_void_p(stream))
        return logits


class LinearHead:
    """A linear head on the encoder's features on the GPU (`d8s_linear`): (N, C) float32 features ->
    (N, K) logits = x W^T + b in float32, on the current stream.  Configuration 4's 1664 -> 8 head after
    the encoder (the reference runs its head right after the encoder on the same device,
    src/knee/infer.py:1015-1017).  There is no CPU path: without the library the call raises."""

    def __init__(self, w, b, device) -> None:
        self.device = torch.device(device)
        self.w = torch.as_tensor(w, dtype=torch.float32).to(self.device).contiguous()
        self.b = torch.as_tensor(b, dtype=torch.float32).to(self.device).contiguous()
        if self.w.dim() != 2 or self.b.shape != (self.w.shape[0],):
            raise ValueError("w must be (K, C) and b (K,)")
        self.K, self.C = self.w.shape
        self._out: torch.Tensor | None = None

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """x (N, C) float32 on the head's device -> logits (N, K) float32, in a buffer of the head's own
        (valid until the next call with as many rows or more)."""
        if x.dim() != 2 or x.shape[1] != self.C or x.dtype != torch.float32 or x.device != self.device:
            raise ValueError(f"x must be (N, {self.C}) float32 on {self.device}")
        x = x.contiguous()
        n = x.shape[0]
        if self._out is None or self._out.shape[0] < n:
            self._out = torch.empty((n, self.K), dtype=torch.float32, device=self.device)
        out = self._out[:n]
        stream = torch.cuda.current_stream(self.device).cuda_stream
        hip.call("d8s_linear", x.data_ptr(), n, self.C, self.w.data_ptr(), self.b.data_ptr(), self.K,
                 out.data_ptr(), ctypes.c_void_p(stream))
        hip.written(out)
        return out
