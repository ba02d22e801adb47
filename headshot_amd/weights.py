"""Converted-checkpoint loading and validation
(crates/headshot-server/src/weights.rs).

A converted checkpoint is a directory holding ``model.safetensors`` and
``manifest.json`` (written by the reference's tools/convert_weights.py).
``Weights.open`` runs every check of ``Weights::open`` (weights.rs:71-95)
before it returns: the manifest names exactly the expected model tree with
the expected shapes, and f32 wherever f32 is mandatory; the file's SHA-256
equals the manifest's ``model_sha256``; the file holds exactly the
manifest's tensors (names, shapes, dtypes). Mismatches raise
``TreeMismatch`` with the full diff, one line per difference, in the
reference's wording (weights.rs:150-175).

The safetensors container is read here directly (an 8-byte little-endian
header length, a JSON header, then the data region), memory-mapped and
validated as the format's own reader does: every tensor's byte range must
match its shape and dtype, and the ranges must tile the data region
exactly. Tensor views are zero-copy numpy arrays over the mapping.

Upload helpers follow model/mod.rs:23-63: ``upload_f32`` (norms, biases,
gammas, always f32 on the device) and ``upload_at`` (GEMM weights and token
constants at the engine precision; an f32-stored tensor is rounded to f16
in f16 mode).
"""
from __future__ import annotations

import hashlib
import json
import mmap
import os
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

DIM = 1024            # trunk / DINO embedding dim (weights.rs:19)
HEAD_IN = 2048        # camera / dense head input dim (weights.rs:21)
DENSE_OC = (256, 512, 1024, 1024)   # DPT pyramid channels (weights.rs:23)
DENSE_FEATURES = 256  # fused-map channels (weights.rs:25)

# safetensors dtype tags and their numpy types / sizes; the checkpoint may
# only hold F16 and F32 (weights.rs:112-119), the rest parse but are refused
_ST_DTYPES = {
    "BOOL": (np.bool_, 1), "U8": (np.uint8, 1), "I8": (np.int8, 1), "F8_E4M3": (np.uint8, 1),
    "F8_E5M2": (np.uint8, 1), "U16": (np.uint16, 2), "I16": (np.int16, 2),
    "F16": (np.float16, 2), "BF16": (np.uint16, 2), "U32": (np.uint32, 4), "I32": (np.int32, 4),
    "F32": (np.float32, 4), "U64": (np.uint64, 8), "I64": (np.int64, 8), "F64": (np.float64, 8),
}
_MANIFEST_DTYPES = {"float16": "F16", "float32": "F32"}


class WeightsError(Exception):
    """weights.rs:27-40 (WeightsError)."""


class WeightsIoError(WeightsError):
    pass


class ManifestParseError(WeightsError):
    pass


class SafeTensorsError(WeightsError):
    pass


class HashMismatch(WeightsError):
    def __init__(self, expected: str, actual: str):
        super().__init__(f"model.safetensors hash mismatch: manifest {expected}, file {actual}")
        self.expected, self.actual = expected, actual


class TreeMismatch(WeightsError):
    def __init__(self, diff: str):
        super().__init__(f"weights do not match the expected model tree:\n{diff}")
        self.diff = diff


@dataclass(frozen=True)
class TensorMeta:
    """Shape and storage dtype ("F16" or "F32") of one tensor
    (weights.rs:51-64)."""
    shape: tuple
    dtype: str

    def __repr__(self) -> str:
        return f"TensorMeta {{ shape: {list(self.shape)}, dtype: {self.dtype} }}"


@dataclass
class Manifest:
    """manifest.json (weights.rs:42-49)."""
    config: object
    checkpoint_sha256: str
    model_sha256: str
    conversion_tool_version: str
    tensors: dict  # name -> TensorMeta

    @staticmethod
    def parse(text: str) -> "Manifest":
        try:
            raw = json.loads(text)
        except ValueError as e:
            raise ManifestParseError(f"manifest parse: {e}") from None

        def need(obj, key, kind):
            if not isinstance(obj, dict) or key not in obj:
                raise ManifestParseError(f"manifest parse: missing field `{key}`")
            v = obj[key]
            if kind is not None and not isinstance(v, kind):
                raise ManifestParseError(f"manifest parse: field `{key}` has the wrong type")
            return v

        tensors = {}
        for name, meta in need(raw, "tensors", dict).items():
            shape = need(meta, "shape", list)
            if not all(isinstance(d, int) and not isinstance(d, bool) and d >= 0 for d in shape):
                raise ManifestParseError(f"manifest parse: {name}: shape must be unsigned integers")
            dt = need(meta, "dtype", str)
            if dt not in _MANIFEST_DTYPES:
                raise ManifestParseError(
                    f"manifest parse: {name}: unknown variant `{dt}`, expected `float16` or `float32`")
            tensors[name] = TensorMeta(tuple(shape), _MANIFEST_DTYPES[dt])
        if "config" not in raw:
            raise ManifestParseError("manifest parse: missing field `config`")
        return Manifest(raw["config"], need(raw, "checkpoint_sha256", str),
                        need(raw, "model_sha256", str), need(raw, "conversion_tool_version", str),
                        tensors)


# ---------------------------------------------------------------------------
# the expected model tree (weights.rs:178-330)

def must_be_f32(name: str) -> bool:
    """Tensors stored f32 whatever the storage precision (weights.rs:185-205):
    norms, gammas, RoPE periods, the token constants, the camera head's last
    linear, the dense head's output projections, and every bias."""
    if ".norm.weight" in name or ".norm.bias" in name:
        return True
    if any(n in name for n in (".norm1.", ".norm2.", ".q_norm.", ".k_norm.", ".token_norm.",
                               ".trunk_norm.")):
        return True
    if name.endswith((".gamma", ".periods", ".bias")):
        return True
    if name in ("aggregator.camera_token", "aggregator.register_token",
                "aggregator.patch_embed.cls_token", "aggregator.patch_embed.storage_tokens"):
        return True
    return name.startswith(("camera_head.camera_branch.2.", "dense_head.proj.",
                            "dense_head.proj_conf."))


def block_tree(prefix: str, dim: int, qk_norm: bool) -> list:
    """One pre-norm block's tensors after conversion (weights.rs:207-236):
    LN1, fused qkv (q | k | v stacked on the output rows), proj, LayerScale
    1, LN2, the 4x MLP, LayerScale 2, and QK-norm over 64 channels when the
    block has it."""
    hidden = 4 * dim
    parts = [("norm1.weight", (dim,)), ("norm1.bias", (dim,)),
             ("attn.qkv.weight", (3 * dim, dim)), ("attn.qkv.bias", (3 * dim,)),
             ("attn.proj.weight", (dim, dim)), ("attn.proj.bias", (dim,)),
             ("ls1.gamma", (dim,)), ("norm2.weight", (dim,)), ("norm2.bias", (dim,)),
             ("mlp.fc1.weight", (hidden, dim)), ("mlp.fc1.bias", (hidden,)),
             ("mlp.fc2.weight", (dim, hidden)), ("mlp.fc2.bias", (dim,)),
             ("ls2.gamma", (dim,))]
    if qk_norm:
        parts += [(f"attn.{n}.{p}", (64,)) for n in ("q_norm", "k_norm") for p in ("weight", "bias")]
    return [(f"{prefix}.{s}", shape) for s, shape in parts]


def trunk_tree(depth: int = 24) -> list:
    """The aggregator trunk's part of the tree (weights.rs:255-261): RoPE
    periods, camera and register tokens, ``depth`` frame / inter-frame block
    pairs with QK-norm."""
    tree = [("aggregator.rope_embed.periods", (16,)),
            ("aggregator.camera_token", (1, 2, 1, DIM)),
            ("aggregator.register_token", (1, 2, 16, DIM))]
    for i in range(depth):
        tree += block_tree(f"aggregator.frame_blocks.{i}", DIM, True)
        tree += block_tree(f"aggregator.inter_frame_blocks.{i}", DIM, True)
    return tree


def expected_tree() -> list:
    """The full post-conversion tree, name -> shape, in the reference's order
    (weights.rs:238-330): DINOv3 ViT-L/16, the aggregator trunk, the camera
    head and the DPT dense head. 1334 tensors (the checkpoint's 1411 keys
    less 76 ``bias_mask`` buffers and the dropped ``mask_token``)."""
    d = "aggregator.patch_embed"
    tree = [(f"{d}.cls_token", (1, 1, DIM)), (f"{d}.storage_tokens", (1, 4, DIM)),
            (f"{d}.patch_embed.proj.weight", (DIM, 3, 16, 16)),
            (f"{d}.patch_embed.proj.bias", (DIM,)), (f"{d}.rope_embed.periods", (16,)),
            (f"{d}.norm.weight", (DIM,)), (f"{d}.norm.bias", (DIM,))]
    for i in range(24):
        tree += block_tree(f"{d}.blocks.{i}", DIM, False)
    tree += trunk_tree(24)

    c = "camera_head"
    tree += [(f"{c}.token_norm.weight", (HEAD_IN,)), (f"{c}.token_norm.bias", (HEAD_IN,)),
             (f"{c}.trunk_norm.weight", (HEAD_IN,)), (f"{c}.trunk_norm.bias", (HEAD_IN,)),
             (f"{c}.camera_branch.0.weight", (DIM, HEAD_IN)), (f"{c}.camera_branch.0.bias", (DIM,)),
             (f"{c}.camera_branch.2.weight", (9, DIM)), (f"{c}.camera_branch.2.bias", (9,))]
    for i in range(4):
        tree += block_tree(f"{c}.trunk.{i}", HEAD_IN, False)

    h = "dense_head"
    tree += [(f"{h}.norm.weight", (HEAD_IN,)), (f"{h}.norm.bias", (HEAD_IN,))]
    for j, oc in enumerate(DENSE_OC):
        tree += [(f"{h}.projects.{j}.weight", (oc, HEAD_IN, 1, 1)), (f"{h}.projects.{j}.bias", (oc,))]
    # resize layers keep each level's channels; level 2 is the identity
    for j, kk in ((0, 4), (1, 2), (3, 3)):
        oc = DENSE_OC[j]
        tree += [(f"{h}.resize_layers.{j}.weight", (oc, oc, kk, kk)),
                 (f"{h}.resize_layers.{j}.bias", (oc,))]
    f = DENSE_FEATURES
    for k in range(1, 5):
        tree.append((f"{h}.scratch.layer{k}_rn.weight", (f, DENSE_OC[k - 1], 3, 3)))
        rn = f"{h}.scratch.refinenet{k}"
        for unit in (("resConfUnit2",) if k == 4 else ("resConfUnit1", "resConfUnit2")):
            for conv in ("conv1", "conv2"):
                tree += [(f"{rn}.{unit}.{conv}.weight", (f, f, 3, 3)),
                         (f"{rn}.{unit}.{conv}.bias", (f,))]
        tree += [(f"{rn}.out_conv.weight", (f, f, 1, 1)), (f"{rn}.out_conv.bias", (f,))]
    for proj in ("proj", "proj_conf"):
        tree += [(f"{h}.{proj}.weight", (16, f, 1, 1)), (f"{h}.{proj}.bias", (16,))]
    return tree


def diff_trees(a_name: str, a: dict, b_name: str, b: dict) -> None:
    """Raise TreeMismatch listing every name missing from ``b``, every
    mismatched entry and every name ``a`` lacks (weights.rs:150-175)."""
    lines = []
    for name in sorted(a):
        if name not in b:
            lines.append(f"missing from {b_name}: {name} {a[name]!r}")
        elif b[name] != a[name]:
            lines.append(f"mismatch {name}: {a_name} {a[name]!r}, {b_name} {b[name]!r}")
    for name in sorted(b):
        if name not in a:
            lines.append(f"unexpected in {b_name}: {name} {b[name]!r}")
    if lines:
        raise TreeMismatch("\n".join(lines) + "\n")


def validate_manifest_tree(manifest: Manifest, tree: list | None = None) -> None:
    """The manifest names exactly ``tree`` (default: the full model,
    ``expected_tree()``) with its shapes; mandatory-f32 tensors must be F32,
    the others may be either, so the manifest's own dtype is expected there
    (F16 if absent) (weights.rs:124-148)."""
    expected = {}
    for name, shape in (expected_tree() if tree is None else tree):
        if must_be_f32(name):
            dt = "F32"
        else:
            m = manifest.tensors.get(name)
            dt = m.dtype if m is not None else "F16"
        expected[name] = TensorMeta(tuple(shape), dt)
    diff_trees("expected", expected, "manifest", manifest.tensors)


# ---------------------------------------------------------------------------
# the safetensors container

class SafeTensorsFile:
    """A memory-mapped safetensors file: ``header`` maps each tensor name to
    (dtype tag, shape, byte offset into the file, byte length);
    ``metadata`` is the optional ``__metadata__`` string map."""

    def __init__(self, path):
        self.path = Path(path)
        try:
            with open(self.path, "rb") as fh:
                size = os.fstat(fh.fileno()).st_size
                self.buf = (mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) if size
                            else b"")
        except OSError as e:
            raise WeightsIoError(f"io: {e}") from None
        self.header, self.metadata = _parse_header(self.buf)

    def names(self) -> list:
        return list(self.header)

    def tensor(self, name: str) -> np.ndarray:
        """Zero-copy read-only view of ``name`` (BF16 and F8 come back as raw
        unsigned integers of the same width)."""
        try:
            tag, shape, off, n = self.header[name]
        except KeyError:
            raise SafeTensorsError(f"safetensors parse: tensor not found: {name}") from None
        dt, _ = _ST_DTYPES[tag]
        count = n // np.dtype(dt).itemsize
        return np.frombuffer(self.buf, dtype=dt, count=count, offset=off).reshape(shape)

    def dtype(self, name: str) -> str:
        return self.header[name][0]

    def sha256(self) -> str:
        return hashlib.sha256(self.buf).hexdigest()


def _parse_header(buf) -> tuple:
    """Validate and decode the header of a safetensors byte buffer."""
    if len(buf) < 8:
        raise SafeTensorsError("safetensors parse: header too small")
    (n,) = struct.unpack_from("<Q", buf, 0)
    if n > len(buf) - 8:
        raise SafeTensorsError("safetensors parse: invalid header length")
    try:
        raw = json.loads(bytes(buf[8:8 + n]).decode("utf-8"))
    except (UnicodeDecodeError, ValueError) as e:
        raise SafeTensorsError(f"safetensors parse: invalid header: {e}") from None
    if not isinstance(raw, dict):
        raise SafeTensorsError("safetensors parse: header is not a JSON object")
    meta = raw.pop("__metadata__", None)
    if meta is not None and not (isinstance(meta, dict)
                                 and all(isinstance(v, str) for v in meta.values())):
        raise SafeTensorsError("safetensors parse: __metadata__ must map strings to strings")
    data0, data_len = 8 + n, len(buf) - 8 - n
    header, spans = {}, []
    for name, info in raw.items():
        try:
            tag, shape, (begin, end) = info["dtype"], info["shape"], info["data_offsets"]
        except (KeyError, TypeError, ValueError):
            raise SafeTensorsError(f"safetensors parse: malformed entry {name}") from None
        if tag not in _ST_DTYPES:
            raise SafeTensorsError(f"safetensors parse: {name}: unknown dtype {tag}")
        if not (isinstance(shape, list) and all(isinstance(d, int) and d >= 0 for d in shape)):
            raise SafeTensorsError(f"safetensors parse: {name}: bad shape")
        if not (isinstance(begin, int) and isinstance(end, int) and 0 <= begin <= end):
            raise SafeTensorsError(f"safetensors parse: {name}: bad data offsets")
        nbytes = int(np.prod(shape, dtype=np.int64)) * _ST_DTYPES[tag][1]
        if end - begin != nbytes:
            raise SafeTensorsError(f"safetensors parse: {name}: {end - begin} bytes for shape "
                                   f"{shape} {tag}")
        header[name] = (tag, tuple(shape), data0 + begin, nbytes)
        spans.append((begin, end, name))
    # the byte ranges must tile the data region with no gap or overlap
    at = 0
    for begin, end, name in sorted(spans):
        if begin != at:
            raise SafeTensorsError(f"safetensors parse: invalid offset for {name}")
        at = end
    if at != data_len:
        raise SafeTensorsError("safetensors parse: data region size does not match the header")
    return header, meta


# ---------------------------------------------------------------------------

class Weights:
    """The converted checkpoint, memory-mapped and fully validated
    (weights.rs:66-122)."""

    def __init__(self, manifest: Manifest, st: SafeTensorsFile):
        self.manifest, self._st = manifest, st

    @staticmethod
    def open(directory, tree: list | None = None) -> "Weights":
        """Open ``manifest.json`` + ``model.safetensors`` from ``directory``
        and run every check (weights.rs:71-95). ``tree`` restricts the
        expected tree (default: the full model); a partial checkpoint such
        as the trunk alone (``trunk_tree``) validates the same way."""
        d = Path(directory)
        try:
            text = (d / "manifest.json").read_text()
        except OSError as e:
            raise WeightsIoError(f"io: {e}") from None
        manifest = Manifest.parse(text)
        validate_manifest_tree(manifest, tree)
        st = SafeTensorsFile(d / "model.safetensors")
        actual = st.sha256()
        if actual != manifest.model_sha256:
            raise HashMismatch(manifest.model_sha256, actual)
        w = Weights(manifest, st)
        w.validate_contents()
        return w

    def validate_contents(self) -> None:
        """The file holds exactly the manifest's tensors: names, shapes and
        dtypes; only F16 and F32 are allowed (weights.rs:104-121)."""
        actual = {}
        for name, (tag, shape, _, _) in self._st.header.items():
            if tag not in ("F16", "F32"):
                raise TreeMismatch(f"{name}: unsupported dtype {tag}")
            actual[name] = TensorMeta(shape, tag)
        diff_trees("manifest", self.manifest.tensors, "file", actual)

    def tensor(self, name: str) -> np.ndarray:
        """A zero-copy numpy view of one tensor (weights.rs:101-103)."""
        return self._st.tensor(name)

    def names(self) -> list:
        return self._st.names()


# ---------------------------------------------------------------------------
# uploads (model/mod.rs:23-70)

def upload_f32(weights: Weights, name: str, device):
    """A parameter as an f32 device tensor, whatever its storage dtype
    (model/mod.rs:23-35)."""
    import torch

    a = weights.tensor(name)
    return torch.from_numpy(np.array(a, dtype=np.float32)).to(device)


def upload_at(weights: Weights, name: str, precision, device):
    """A GEMM weight or token constant at the engine precision
    (model/mod.rs:44-63): f16 mode keeps f16-stored tensors and rounds
    f32-stored ones to f16 (round to nearest even); f32 mode widens."""
    import torch

    if precision == torch.float32:
        return upload_f32(weights, name, device)
    if precision != torch.float16:
        raise ValueError(f"{name}: unsupported precision {precision}")
    a = weights.tensor(name)
    return torch.from_numpy(np.array(a, dtype=np.float16)).to(device)


def read_f32(weights: Weights, name: str) -> np.ndarray:
    """A small f32 tensor on the host, e.g. RoPE periods (model/mod.rs:65-70)."""
    a = weights.tensor(name)
    if a.dtype != np.float32:
        raise WeightsError(f"{name}: expected f32")
    return np.array(a)
