"""Packages from trained weights: a `KneeBaseline` checkpoint -> the INT8 encoder package.

The reference builds its packages from the training checkpoints `fold{seed}.pt`
(`kaggle/int8_pack/pack_dense8s.py:485-487,1228-1257` -> `src/knee/aggregate.py:137-167`
`model_from_checkpoint`): the DenseNet169 under `encoder.*` of the `KneeBaseline` state dict is
calibrated on windows, planned, saved, reloaded and gated against its float32 forward.  The same steps
here, with the checkpoint read by `torch.load(weights_only=True)` (tensors and plain containers only;
nothing in the file is executed) and the encoder rebuilt as `densenet.DenseNet` from its keys alone, so
neither the reference's model classes nor its configuration code are needed:

- `load_checkpoint(path)`          {"cfg": dict, "model": state dict} (a bare state dict is accepted);
- `encoder_from_state(sd)`         the `densenet.DenseNet` of the `encoder.features.*` entries;
- `input_norm(cfg)`                the (mean, std) the encoder's windows are normalised with;
- `build_pack(ckpt, cal_batches, n, img)`  calibrate -> plan -> package (in memory, or saved);
- `gate(pack, model, x)`           the reloaded package's features against the float32 forward, the
                                   reference's check before a package is used.

    python -m rsna_knee_efficiency_amd.checkpoint fold0.pt --cal windows.npy --n 96 --out pack.npz

(`windows.npy`: uint8 calibration windows (N, 3, img, img); the reference calibrates on 64 studies'
windows.)  The head's weights are in the same state dict: `head.KneeHead(ck["model"], device)`.
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path

import numpy as np
import torch

from . import dense8s, densenet

ENCODER_PREFIX = "encoder."
# prefixes a training wrapper may put in front of every key (torch.compile, DistributedDataParallel)
WRAPPER_PREFIXES = ("_orig_mod.", "module.")
IMAGENET_MEAN = (0.485, 0.456, 0.406)       # `input_norm: imagenet` (src/knee/models/baseline.py:62-64)
IMAGENET_STD = (0.229, 0.224, 0.225)


def load_checkpoint(path) -> dict:
    """The checkpoint at `path` as {"cfg": dict, "model": state dict}, loaded with weights_only=True
    (a file holding anything but tensors and plain containers is refused by torch, not executed)."""
    ck = torch.load(Path(path), map_location="cpu", weights_only=True)
    if not isinstance(ck, dict):
        raise ValueError(f"{path}: a dict checkpoint expected, got {type(ck).__name__}")
    if "model" in ck and isinstance(ck["model"], dict):
        return {"cfg": ck.get("cfg") or {}, "model": ck["model"]}
    if all(isinstance(v, torch.Tensor) for v in ck.values()):
        return {"cfg": {}, "model": ck}
    raise ValueError(f"{path}: no 'model' state dict in the checkpoint (keys {sorted(ck)[:6]})")


def _strip(sd: dict) -> dict:
    out = {}
    for k, v in sd.items():
        for p in WRAPPER_PREFIXES:
            if k.startswith(p):
                k = k[len(p):]
        out[k] = v
    return out


def encoder_state(sd: dict) -> dict:
    """The encoder's `features.*` entries of a `KneeBaseline` state dict (keys `encoder.features.*`),
    or of a bare DenseNet state dict (keys `features.*`)."""
    sd = _strip(sd)
    enc = {k[len(ENCODER_PREFIX):]: v for k, v in sd.items()
           if k.startswith(ENCODER_PREFIX + "features.")}
    if not enc:
        enc = {k: v for k, v in sd.items() if k.startswith("features.")}
    if not enc:
        raise ValueError("no encoder weights: expected keys 'encoder.features.*' or 'features.*'")
    if any(k.startswith(ENCODER_PREFIX) and not k.startswith(ENCODER_PREFIX + "features.")
           and not k.endswith("num_batches_tracked") for k in sd):
        extra = sorted(k for k in sd if k.startswith(ENCODER_PREFIX) and "features." not in k)
        raise ValueError(f"encoder entries outside features: {extra[:4]} (not a DenseNet encoder)")
    return enc


def block_config(enc: dict) -> tuple[int, ...]:
    """Layers per dense block, read from the keys `features.denseblock{k}.denselayer{j}.*`."""
    blocks = []
    while True:
        k = len(blocks) + 1
        n = 0
        while f"features.denseblock{k}.denselayer{n + 1}.conv1.weight" in enc:
            n += 1
        if n == 0:
            return tuple(blocks)
        blocks.append(n)


def encoder_from_state(sd: dict) -> densenet.DenseNet:
    """A `densenet.DenseNet` in eval holding the encoder weights of `sd` (every key checked: a missing
    or unexpected one raises, as `load_state_dict(strict=True)`)."""
    enc = encoder_state(sd)
    blocks = block_config(enc)
    if not blocks:
        raise ValueError("no dense blocks in the encoder weights")
    in_chans = int(enc["features.conv0.weight"].shape[1])
    model = densenet.DenseNet(blocks, in_chans=in_chans)
    model.load_state_dict({k: v.float() if v.is_floating_point() else v for k, v in enc.items()},
                          strict=True)
    return model.eval()


def input_norm(cfg: dict) -> tuple[tuple[float, ...], tuple[float, ...]]:
    """(mean, std) of the encoder's input: windows u / 255 as they are (mean 0, std 1), unless the
    model was trained with `input_norm: imagenet` (src/knee/models/baseline.py:556-566)."""
    norm = ((cfg or {}).get("model") or {}).get("input_norm")
    if norm is None:
        return (0.0, 0.0, 0.0), (1.0, 1.0, 1.0)
    if norm == "imagenet":
        return IMAGENET_MEAN, IMAGENET_STD
    raise ValueError(f"input_norm {norm!r}: expected None or 'imagenet'")


def image_size(cfg: dict, default: int = 512) -> int:
    return int(((cfg or {}).get("cache") or {}).get("img", default))


def normalised(u8: torch.Tensor, mean, std) -> torch.Tensor:
    """uint8 windows (N, 3, H, W) -> the float input (u / 255 - mean_c) / std_c."""
    m = torch.tensor(mean, dtype=torch.float32, device=u8.device).view(1, -1, 1, 1)
    s = torch.tensor(std, dtype=torch.float32, device=u8.device).view(1, -1, 1, 1)
    return (u8.float() / 255.0 - m) / s


def build_pack(ckpt, cal_batches, n: int, img: int | None = None, device=None, out=None) -> dict:
    """The package of a checkpoint (a path or a `load_checkpoint` dict): the encoder calibrated on
    `cal_batches` (uint8 windows (N, 3, img, img), normalised as the model's cfg says), planned at
    `img` (default: the cfg's cache side) for `n` images per pass, with uint8 input.  Saved to `out`
    when given.  Returns {"pack", "plan", "cal", "model" (the float encoder, CPU), "mean", "std"}."""
    ck = load_checkpoint(ckpt) if isinstance(ckpt, (str, Path)) else ckpt
    model = encoder_from_state(ck["model"])
    mean, std = input_norm(ck.get("cfg"))
    img = int(img or image_size(ck.get("cfg")))
    dev = torch.device(device) if device is not None else torch.device("cpu")
    model.to(dev)
    try:
        cal = dense8s.calibrate(model, [normalised(torch.as_tensor(b).to(dev), mean, std)
                                        for b in cal_batches])
    finally:
        model.cpu()
    plan = dense8s.make_plan(model, cal, img)
    kw = {"input_kind": "u8", "mean": mean, "std": std}
    if out is not None:
        dense8s.save_pack(Path(out), plan, n, **kw)
    return {"pack": dense8s.make_pack(plan, n, **kw), "plan": plan, "cal": cal, "model": model,
            "mean": mean, "std": std}


@torch.no_grad()
def gate(pack: dict, model: densenet.DenseNet, x_u8: torch.Tensor, mean, std, chunk: int = 16) -> dict:
    """The package's features on uint8 windows `x_u8` (on the GPU) against the float32 encoder's:
    max-abs, rel_l2, minimum cosine, and `ok` under the reference's gate (rel_l2 <= 1.05 x 0.067,
    `kaggle/int8_pack/pack_dense8s.py:839-842,1151`; cosine >= 0.99)."""
    dev = x_u8.device
    enc = dense8s.Dense8SEncoder(pack, dev.index or 0, x_u8.shape[0])
    got = enc(x_u8).double().cpu().numpy()
    model = model.to(dev).eval()
    try:
        ref = torch.cat([model(normalised(c, mean, std)) for c in x_u8.split(chunk)]).double().cpu().numpy()
    finally:
        model.cpu()
    cos = (got * ref).sum(1) / np.maximum(np.linalg.norm(got, axis=1) * np.linalg.norm(ref, axis=1), 1e-30)
    res = {"max_abs": float(np.abs(got - ref).max()),
           "rel_l2": float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)),
           "cos_min": float(cos.min())}
    res["ok"] = bool(res["rel_l2"] <= 1.05 * 0.067 and res["cos_min"] >= 0.99)
    return res


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description="INT8 encoder package from a KneeBaseline checkpoint")
    ap.add_argument("checkpoint")
    ap.add_argument("--cal", required=True, help="uint8 calibration windows (N, 3, img, img), .npy")
    ap.add_argument("--n", type=int, default=96, help="images per pass (graph batch)")
    ap.add_argument("--img", type=int, default=None)
    ap.add_argument("--out", required=True)
    ap.add_argument("--batch", type=int, default=8, help="calibration windows per forward")
    args = ap.parse_args(argv)
    x = np.load(args.cal, allow_pickle=False)
    if x.dtype != np.uint8 or x.ndim != 4 or x.shape[1] != 3:
        raise SystemExit(f"{args.cal}: uint8 (N, 3, img, img) expected, got {x.dtype} {x.shape}")
    dev = "cuda:0" if torch.cuda.is_available() else "cpu"
    batches = [torch.from_numpy(b) for b in np.array_split(x, max(1, -(-len(x) // args.batch)))]
    res = build_pack(args.checkpoint, batches, args.n, args.img, device=dev, out=args.out)
    report = {"out": args.out, "n": args.n, "img": res["plan"].img, "mean": res["mean"], "std": res["std"]}
    if dev != "cpu":
        pk = dense8s.load_pack(Path(args.out))
        sample = torch.from_numpy(x[:min(len(x), args.n)]).to(dev)
        report["gate"] = gate(pk, res["model"], sample, res["mean"], res["std"])
    print(json.dumps(report))


if __name__ == "__main__":
    main()
