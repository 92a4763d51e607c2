"""Integer checkpoint I/O in the reference's "i-whisper-int" v1 format
(i_whisper/__init__.py:248-493).

On disk a model is a directory ``<prefix>/iwhisper-<model_name>/`` holding

* ``config.json``: ``{"format": "i-whisper-int", "format_version": 1,
  "model_name": ..., "dims": {ModelDimensions fields}}`` (__init__.py:304-309);
* ``model.safetensors``: the ``Whisper_int`` state dict (reference keys and
  integer dtypes, contiguous CPU tensors) with the metadata
  ``{"format": "i-whisper-int", "format_version": "1"}`` (__init__.py:313-326).

A checkpoint the reference exported loads here strictly (same keys, shapes and
dtypes), and one saved here loads in the reference. Reading uses safetensors
only, which executes nothing from the file.
"""
from __future__ import annotations

import json
from dataclasses import asdict
from pathlib import Path
from typing import Callable, Optional, Union

import torch
from safetensors.torch import load_file, save_file

from .model_int import ModelDimensions, Whisper_int

INT_FORMAT = "i-whisper-int"
INT_FORMAT_VERSION = 1
INT_CKPT_ROOT = Path("CKPT")


def resolve_int_model_dir(name: Union[str, Path], root: Union[str, Path] = INT_CKPT_ROOT) -> Path:
    """A model directory, a path to its model.safetensors, or an alias
    ("base" -> <root>/iwhisper-base), as __init__.py:253-278 resolves them."""
    path = Path(name)
    if path.is_dir():
        return path
    if path.is_file():
        if path.name != "model.safetensors":
            raise RuntimeError(f"Expected model.safetensors, got: {path}")
        return path.parent
    model_dir = Path(root) / f"iwhisper-{name}"
    if model_dir.is_dir():
        return model_dir
    raise RuntimeError(f"I-Whisper INT model '{name}' not found. Expected directory: {model_dir}")


def save_int_model(model: Whisper_int, prefix: Union[str, Path], model_name: str) -> Path:
    """Write ``model`` as <prefix>/iwhisper-<model_name>/ (__init__.py:281-334).
    Returns the model directory."""
    if not isinstance(model, Whisper_int):
        raise TypeError("model must be an instance of Whisper_int")
    model_dir = Path(prefix) / f"iwhisper-{model_name}"
    model_dir.mkdir(parents=True, exist_ok=True)
    config = {
        "format": INT_FORMAT,
        "format_version": INT_FORMAT_VERSION,
        "model_name": model_name,
        "dims": asdict(model.dims),
    }
    state = {k: v.detach().cpu().contiguous() for k, v in model.state_dict().items()}
    save_file(state, str(model_dir / "model.safetensors"),
              metadata={"format": INT_FORMAT, "format_version": str(INT_FORMAT_VERSION)})
    with open(model_dir / "config.json", "w", encoding="utf-8") as f:
        json.dump(config, f, indent=2)
    return model_dir


def _read_checked(model_dir: Path):
    config_path = model_dir / "config.json"
    tensor_path = model_dir / "model.safetensors"
    if not config_path.is_file():
        raise RuntimeError(f"Missing model configuration: {config_path}")
    if not tensor_path.is_file():
        raise RuntimeError(f"Missing model tensors: {tensor_path}")
    with open(config_path, "r", encoding="utf-8") as f:
        config = json.load(f)
    if config.get("format") != INT_FORMAT:
        raise RuntimeError(f"Unsupported model format: {config.get('format')}")
    if config.get("format_version") != INT_FORMAT_VERSION:
        raise RuntimeError(f"Unsupported model format version: {config.get('format_version')}")
    return ModelDimensions(**config["dims"]), load_file(str(tensor_path), device="cpu")


def load_int_model(name: Union[str, Path], device: Optional[Union[str, torch.device]] = None,
                   root: Union[str, Path] = INT_CKPT_ROOT) -> Whisper_int:
    """Load a checkpoint into ``Whisper_int`` with a strict state-dict match
    (__init__.py:338-413). ``device`` defaults to the GPU when one is present."""
    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    dims, state = _read_checked(resolve_int_model_dir(name, root))
    model = Whisper_int(dims)
    model.load_state_dict(state, strict=True)
    del state
    return model.to(device).eval()


def load_int_params(name: Union[str, Path], root: Union[str, Path] = INT_CKPT_ROOT):
    """(dims, {state-dict key: numpy array}) of a checkpoint, without building
    the model (the form ``Whisper_int.from_params`` takes)."""
    dims, state = _read_checked(resolve_int_model_dir(name, root))
    return dims, {k: v.numpy() for k, v in state.items()}


def _exact_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    # torch.equal has no kernels for uint16/uint32 (__init__.py:416-428)
    if a.dtype in (torch.uint16, torch.uint32):
        return torch.equal(a.to(torch.int64), b.to(torch.int64))
    return torch.equal(a, b)


def verify_int_model_roundtrip(original: Whisper_int, loaded: Whisper_int,
                               streamer: Optional[Callable[[str], None]] = None) -> None:
    """Keys, dtypes, shapes and values of two models' persistent state are
    identical, else AssertionError (__init__.py:431-493)."""
    if streamer is None:
        streamer = print
    sa, sb = original.state_dict(), loaded.state_dict()
    if sa.keys() != sb.keys():
        missing, unexpected = sa.keys() - sb.keys(), sb.keys() - sa.keys()
        if missing:
            streamer(f"Missing keys: {sorted(missing)}")
        if unexpected:
            streamer(f"Unexpected keys: {sorted(unexpected)}")
        raise AssertionError("State dict keys mismatch")
    for name in sa:
        a, b = sa[name].detach().cpu(), sb[name].detach().cpu()
        if a.dtype != b.dtype:
            raise AssertionError(f"{name}: dtype mismatch: {a.dtype} != {b.dtype}")
        if a.shape != b.shape:
            raise AssertionError(f"{name}: shape mismatch: {a.shape} != {b.shape}")
        if not _exact_equal(a, b):
            raise AssertionError(f"{name}: tensor value mismatch")
    streamer(f"Integer model round-trip verification passed ({len(sa)} tensors checked)")

