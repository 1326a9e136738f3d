"""The INT8 pipeline in float64 PyTorch: the reference's own CPU path, restated.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Follows `emulate` of `src/knee/dense8s.py:549-622`
for the reference's final configuration: every prologue in fp16 (`f16_layers` = all layers and
transitions, the `w64_pl` conv1 and `trans_w*` transitions), the u8 bottleneck of "our" conv2
(`conv2="ours"`), the transition in its integer form (sum of the four accumulators of the 2x2 square,
`dense8s.py:605-617`), norm5 + ReLU + mean.  Integer sums are exact in float64.

Differences from the kernels (and from `oracle/lib.py`, which reproduces the kernels bit for bit) are
the epilogue roundings: here the products with the float32 tables are rounded once in float64, there
in float32; bytes may differ by one where a value falls within a float32 ulp of a rounding boundary.

The fp16 rounding of the prologue is done by numpy's float64 -> float16 conversion (one rounding):
`torch`'s CPU conversion goes through float32 and can round twice.

Stems: "fp" = the reference's float stem (`dense8s.py:574-578`: conv with S_w0, S_b0 = norm0 and 1 /
sigma0 folded in, ReLU, max-pool, round); "f16" = this build's stem formula (fp16 weights S_w16 on the
fp16 input values, bias, ReLU, times 1 / sigma0, round, max-pool) with the sum in float64.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

QU, QS, GROWTH, BOTTLENECK = 255, 127, 32, 128


def f16_round(t: torch.Tensor) -> torch.Tensor:
    """Nearest fp16 value of every element (float64 in, float64 out, one rounding)."""
    return torch.from_numpy(t.detach().cpu().numpy().astype(np.float16).astype(np.float64))


def abh_values(abh: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    h = np.ascontiguousarray(abh).view(np.float16).astype(np.float64)
    return h[:, :2].reshape(-1), h[:, 2:].reshape(-1)


def _rq(t, lo, hi, quant):
    return torch.round(t).clamp(lo, hi) if quant else t


@torch.no_grad()
def prologue(X: torch.Tensor, abh: np.ndarray, ab: np.ndarray, quant: bool) -> torch.Tensor:
    """u = RNE(255 sat(fp16(A q + B))) (quant) or relu(a x + b) 255 (not quant)."""
    col = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.float64).view(1, -1, 1, 1)  # noqa: E731
    if quant:
        a16, b16 = abh_values(abh)
        t = col(a16) * X + col(b16)
        return torch.round(f16_round(t).clamp(0, 1) * QU)
    t = col(ab[:, 0]) * X + col(ab[:, 1])
    return t.clamp_min(0) * QU


@torch.no_grad()
def stem(plan, par: dict, x: torch.Tensor, quant: bool = True, kind: str = "fp") -> torch.Tensor:
    """The block-0 store (N, 64, H/4, W/4) as float64 integers."""
    T = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.float64)  # noqa: E731
    x = x.double()
    if kind == "fp":
        y = F.relu(F.conv2d(x, T(par["S_w0"]), T(par["S_b0"]), stride=2, padding=3))
        return _rq(F.max_pool2d(y, 3, 2, 1), -QS, QS, quant)
    w16 = T(np.asarray(par["S_w16"]).view(np.float16).astype(np.float64)).view(64, 3, 7, 8)[..., 1:]
    y = F.conv2d(x, w16.contiguous(), stride=2, padding=3) + T(par["S_bias"]).view(1, -1, 1, 1)
    t = F.relu(y) * T(par["S_inv"]).view(1, -1, 1, 1)
    q = torch.round(t.clamp(max=QS)) if quant else t
    return F.max_pool2d(q, 3, 2, 1)


@torch.no_grad()
def emulate(plan, x: torch.Tensor, par: dict, quant: bool = True, stem_kind: str = "fp",
            trace: dict | None = None, q0: torch.Tensor | None = None) -> torch.Tensor:
    """Features (N, n_features) float32 of the INT8 pipeline on x (N, 3, H, W), on the CPU in float64.
    `plan` is a `dense8s.SPlan` (integer weights), `par` its `kernel_params`.  `trace` receives the
    store {(block, j): tensor}; `q0` replaces the stem output (the block-0 store) when given.
    `quant=False`: no roundings or saturations (the ReLUs stay): the encoder with only its weights
    quantised (`src/knee/dense8s.py:557-559`)."""
    trace = {} if trace is None else trace
    T = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.float64)  # noqa: E731
    col = lambda a: T(a).view(1, -1, 1, 1)  # noqa: E731
    q = stem(plan, par, x, quant, stem_kind) if q0 is None else q0.double()
    for bi, blk in enumerate(plan.blocks):
        store = [q]
        trace[(bi, 0)] = q
        for li, L in enumerate(blk.layers):
            X = torch.cat(store, 1)
            u = prologue(X, par[f"L{bi}_{li}_abh"], par[f"L{bi}_{li}_ab"], quant)
            acc = F.conv2d(u, T(L.w1.astype(np.float64)).view(BOTTLENECK, -1, 1, 1))
            gd = par[f"L{bi}_{li}_gdu"]
            t = col(gd[:, 0]) * acc + col(gd[:, 1])
            v = torch.round(t.clamp(0, 1) * QU) if quant else t.clamp_min(0) * QU
            trace[("bott", bi, li)] = v
            acc2 = F.conv2d(v, T(L.w2.astype(np.float64)), padding=1)
            c2 = torch.as_tensor(par[f"L{bi}_{li}_c2u"], dtype=torch.float32).double()
            seg = acc2 * c2.view(1, -1, 1, 1)
            if quant:
                seg = torch.round(seg).clamp(-QS, QS)
            store.append(seg)
            trace[(bi, li + 1)] = seg
        X = torch.cat(store, 1)
        if blk.ta is not None:
            u = prologue(X, par[f"T{bi}_abh"], par[f"T{bi}_ab"], quant)
            acc = F.conv2d(u, T(blk.tw.astype(np.float64)).view(blk.tw.shape[0], -1, 1, 1))
            s4 = F.avg_pool2d(acc, 2) * 4
            k = col(par[f"T{bi}_gd"][:, 0])
            q = torch.round(k * s4).clamp(-QS, QS) if quant else k * s4
        else:
            ab = par["F_ab"]
            z = F.relu(col(ab[:, 0]) * X + col(ab[:, 1]))
            return z.mean(dim=(2, 3)).float()
    raise RuntimeError("plan without a final block")


@torch.no_grad()
def weight_quant_state(sd: dict) -> dict:
    """The state_dict with every conv weight but the stem's rounded to int8 per output channel, as the
    plan does (`src/knee/dense8s.py:646-657`): the float reference of `emulate(quant=False)`."""
    out = {}
    for k, v in sd.items():
        if k.endswith(".weight") and v.dim() == 4 and not k.startswith("features.conv0"):
            w = v.detach().float()
            scale = w.abs().flatten(1).amax(1).clamp_min(1e-12) / QS
            inv = (1.0 / scale).view(-1, 1, 1, 1)
            q = torch.round(w * inv).clamp(-128, 127)
            out[k] = q * scale.view(-1, 1, 1, 1)
        else:
            out[k] = v
    return out
