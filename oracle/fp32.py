"""The float32 DenseNet forward, written functionally from a timm-layout state_dict.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the parity reference of the INT8 features and the
CPU baseline of bench.py.  It is a second, independent writing of the network of
`src/knee/models/densenet.py:27-104` (conv0 7x7/2 -> norm0 -> ReLU -> maxpool 3x3/2; dense layers
BN-ReLU-1x1(128)-BN-ReLU-3x3(32) over the concatenation; transitions BN-ReLU-1x1(c/2)-avgpool 2x2;
norm5 -> ReLU -> global mean), so a mistake in the package's `densenet.DenseNet` module would show as
a disagreement between the two.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

EPS = 1e-5


def _bn(x, sd, p):
    return F.batch_norm(x, sd[p + ".running_mean"], sd[p + ".running_var"], sd[p + ".weight"],
                        sd[p + ".bias"], False, 0.0, EPS)


def block_config(sd) -> tuple[int, ...]:
    out, k = [], 1
    while any(key.startswith(f"features.denseblock{k}.") for key in sd):
        n = 0
        while f"features.denseblock{k}.denselayer{n + 1}.conv1.weight" in sd:
            n += 1
        out.append(n)
        k += 1
    return tuple(out)


@torch.no_grad()
def forward(sd: dict, x: torch.Tensor, tap=None) -> torch.Tensor:
    """Features (B, C) of the float32 input x (B, 3, H, W).  `tap(name, tensor)`, if given, sees the
    intermediates the INT8 plan quantises: "pool0" (block 0's input), "relu1.{b}.{l}" / "relu2.{b}.{l}"
    (the inputs of conv1 / conv2 of layer l of block b), "conv2.{b}.{l}" (its 32 new channels),
    "trelu.{b}" (the transition conv's input) and "tpool.{b}" (block b + 1's input)."""
    sd = {k: v.float() for k, v in sd.items()}
    tap = tap or (lambda name, t: None)
    x = x.float()
    y = F.conv2d(x, sd["features.conv0.weight"], stride=2, padding=3)
    y = F.max_pool2d(F.relu(_bn(y, sd, "features.norm0")), 3, 2, 1)
    tap("pool0", y)
    blocks = block_config(sd)
    for k, n_layers in enumerate(blocks, start=1):
        feats = [y]
        for j in range(1, n_layers + 1):
            p = f"features.denseblock{k}.denselayer{j}"
            z = F.relu(_bn(torch.cat(feats, 1), sd, p + ".norm1"))
            tap(f"relu1.{k - 1}.{j - 1}", z)
            z = F.conv2d(z, sd[p + ".conv1.weight"])
            z = F.relu(_bn(z, sd, p + ".norm2"))
            tap(f"relu2.{k - 1}.{j - 1}", z)
            feats.append(F.conv2d(z, sd[p + ".conv2.weight"], padding=1))
            tap(f"conv2.{k - 1}.{j - 1}", feats[-1])
        y = torch.cat(feats, 1)
        if k < len(blocks):
            p = f"features.transition{k}"
            z = F.relu(_bn(y, sd, p + ".norm"))
            tap(f"trelu.{k - 1}", z)
            y = F.avg_pool2d(F.conv2d(z, sd[p + ".conv.weight"]), 2)
            tap(f"tpool.{k - 1}", y)
    return F.relu(_bn(y, sd, "features.norm5")).mean(dim=(2, 3))
