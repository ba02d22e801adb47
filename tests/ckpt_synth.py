"""Synthetic converted checkpoints for the loader and trunk tests.

``write_checkpoint`` writes ``model.safetensors`` with the safetensors
library's own writer (so the package's reader is checked against an
independent implementation of the format) and a ``manifest.json`` in the
converter's layout (weights.rs:42-64): config, checkpoint and file SHA-256,
tool version, and each tensor's shape and dtype ("float16" / "float32").

Values follow the reference checkpoints' kinds: LayerNorm weights ~N(1,
.02), biases ~N(0, .02), linear weights ~N(0, 1/fan_in), LayerScale gammas
~N(0, ``ls``) , tokens ~N(0, 1), RoPE periods 100^(2i/32).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
from safetensors.numpy import save_file


def synth_values(tree, seed: int, f32_names=(), ls: float = 0.05) -> dict:
    """name -> array for every (name, shape) of ``tree``: tensors that must
    be f32 (and those in ``f32_names``) as float32, the rest float16."""
    from headshot_amd.weights import must_be_f32

    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in tree:
        if name.endswith(".periods"):
            a = (100.0 ** (2.0 * np.arange(16) / 32.0)).astype(np.float32)
        elif name.endswith("norm1.weight") or name.endswith("norm2.weight") or "_norm.weight" in name \
                or name.endswith(".norm.weight"):
            a = 1.0 + 0.02 * rng.standard_normal(shape)
        elif name.endswith(".gamma"):
            a = ls * rng.standard_normal(shape)
        elif name.endswith(".bias"):
            a = 0.02 * rng.standard_normal(shape)
        elif name.endswith("_token") or name.endswith("storage_tokens"):
            a = rng.standard_normal(shape)
        else:
            a = rng.standard_normal(shape, dtype=np.float32) / np.sqrt(shape[-1] if len(shape) == 2
                                                                     else np.prod(shape[1:]))
        f32 = must_be_f32(name) or name in f32_names
        out[name] = np.ascontiguousarray(a, dtype=np.float32 if f32 else np.float16)
    return out


def write_checkpoint(directory, values: dict, manifest_overrides=None) -> Path:
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    path = d / "model.safetensors"
    save_file(values, str(path))
    sha = hashlib.sha256(path.read_bytes()).hexdigest()
    manifest = {
        "config": {"synthetic": True},
        "checkpoint_sha256": "",
        "model_sha256": sha,
        "conversion_tool_version": "synthetic",
        "tensors": {n: {"shape": list(a.shape),
                        "dtype": "float32" if a.dtype == np.float32 else "float16"}
                    for n, a in values.items()},
    }
    manifest.update(manifest_overrides or {})
    (d / "manifest.json").write_text(json.dumps(manifest))
    return d
