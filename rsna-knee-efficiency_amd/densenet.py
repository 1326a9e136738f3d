"""DenseNet169 in timm / torchvision layout, in plain PyTorch: the float model the INT8 plan is built from.

The module names and the state_dict keys are those of `timm.create_model("densenet169",
num_classes=0)` (features.conv0, features.norm0, features.pool0, features.denseblock{k}.denselayer{j}
.{norm1, conv1, norm2, conv2}, features.transition{k}.{norm, conv, pool}, features.norm5), as in the
reference's hand-written copy `src/knee/models/densenet.py:20-114`: checkpoints load unchanged and
`dense8s.calibrate` walks the same modules.  Growth 32, bottleneck 4 x 32, blocks 6/12/32/32,
transitions halve the channels, 1664 output features.

`seeded_densenet169(seed)` gives the synthetic weights of the benchmark configurations: He-normal
convolutions (std sqrt(2 / fan_in)), BatchNorm gamma ~ U(0.8, 1.2), beta ~ N(0, 0.1),
running_mean ~ N(0, 0.1), running_var ~ U(0.5, 1.5).
"""
from __future__ import annotations

import math
from collections import OrderedDict

import torch
import torch.nn as nn
import torch.nn.functional as F

GROWTH = 32
BN_SIZE = 4
STEM_CHANNELS = 64
BLOCKS = {"densenet121": (6, 12, 24, 16), "densenet169": (6, 12, 32, 32)}


class DenseLayer(nn.Module):
    """BN-ReLU-1x1 (to 128) then BN-ReLU-3x3 (to 32) over the concatenation of the earlier features."""

    def __init__(self, c_in: int) -> None:
        super().__init__()
        mid = BN_SIZE * GROWTH
        self.norm1 = nn.BatchNorm2d(c_in)
        self.relu1 = nn.ReLU()
        self.conv1 = nn.Conv2d(c_in, mid, 1, bias=False)
        self.norm2 = nn.BatchNorm2d(mid)
        self.relu2 = nn.ReLU()
        self.conv2 = nn.Conv2d(mid, GROWTH, 3, padding=1, bias=False)

    def forward(self, feats: list[torch.Tensor]) -> torch.Tensor:
        x = torch.cat(feats, 1)
        x = self.conv1(self.relu1(self.norm1(x)))
        return self.conv2(self.relu2(self.norm2(x)))


class DenseBlock(nn.ModuleDict):
    def __init__(self, n_layers: int, c_in: int) -> None:
        super().__init__({f"denselayer{i + 1}": DenseLayer(c_in + i * GROWTH)
                          for i in range(n_layers)})

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        feats = [x]
        for layer in self.values():
            feats.append(layer(feats))
        return torch.cat(feats, 1)


class Transition(nn.Sequential):
    def __init__(self, c_in: int, c_out: int) -> None:
        super().__init__(OrderedDict(norm=nn.BatchNorm2d(c_in), relu=nn.ReLU(),
                                     conv=nn.Conv2d(c_in, c_out, 1, bias=False),
                                     pool=nn.AvgPool2d(2, 2)))


class DenseNet(nn.Module):
    """`forward(x)`: (B, in_chans, H, W) -> (B, C) global features, C = 1664 for the 169."""

    def __init__(self, blocks: tuple[int, ...] = BLOCKS["densenet169"], in_chans: int = 3) -> None:
        super().__init__()
        layers: OrderedDict[str, nn.Module] = OrderedDict(
            conv0=nn.Conv2d(in_chans, STEM_CHANNELS, 7, stride=2, padding=3, bias=False),
            norm0=nn.BatchNorm2d(STEM_CHANNELS), relu0=nn.ReLU(),
            pool0=nn.MaxPool2d(3, stride=2, padding=1))
        c = STEM_CHANNELS
        for k, n_layers in enumerate(blocks, start=1):
            layers[f"denseblock{k}"] = DenseBlock(n_layers, c)
            c += n_layers * GROWTH
            if k < len(blocks):
                layers[f"transition{k}"] = Transition(c, c // 2)
                c //= 2
        layers["norm5"] = nn.BatchNorm2d(c)
        self.features = nn.Sequential(layers)
        self.num_features = c

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.relu(self.features(x)).mean(dim=(2, 3))


def densenet169(in_chans: int = 3) -> DenseNet:
    return DenseNet(BLOCKS["densenet169"], in_chans)


@torch.no_grad()
def seeded_init_(model: nn.Module, seed: int) -> nn.Module:
    """Synthetic weights (He-normal convs, the BatchNorm distributions of the module docstring), drawn
    from one CPU generator in module order: the same seed gives the same model everywhere.
    """
    g = torch.Generator().manual_seed(int(seed))
    for mod in model.modules():
        if isinstance(mod, nn.Conv2d):
            fan_in = mod.in_channels * mod.kernel_size[0] * mod.kernel_size[1]
            w = torch.randn(mod.weight.shape, generator=g, dtype=torch.float32)
            mod.weight.copy_(w * math.sqrt(2.0 / fan_in))
        elif isinstance(mod, nn.BatchNorm2d):
            n = mod.num_features
            mod.weight.copy_(0.8 + 0.4 * torch.rand(n, generator=g))
            mod.bias.copy_(0.1 * torch.randn(n, generator=g))
            mod.running_mean.copy_(0.1 * torch.randn(n, generator=g))
            mod.running_var.copy_(0.5 + torch.rand(n, generator=g))
    return model.eval()


def seeded_densenet169(seed: int, blocks: tuple[int, ...] = BLOCKS["densenet169"]) -> DenseNet:
    return seeded_init_(DenseNet(blocks), seed)
