"""Converted-checkpoint loading (headshot_amd.weights; weights.rs) and the
reference-dump reader (headshot_amd.parity.Dump; parity.rs), on the CPU.

Pins: the reference's own tests of weights.rs (weights.rs:332-441: tree
size 1334 and uniqueness, a full fake manifest validates, the diff reports
all four mismatch kinds in exactly four lines, hash and contents checks)
restated here; the tree's size re-derived independently from the model's
structure; the safetensors reader checked against the safetensors
library's writer and reader on random files, and on malformed files the
library also refuses.
"""
import json
import struct

import numpy as np
import pytest
import safetensors.numpy as stn
import torch

from headshot_amd import weights as W
from headshot_amd.parity import Dump, fixtures_dir
from tests.ckpt_synth import synth_values, write_checkpoint


def full_fake_tensors():
    """weights.rs:348-361: f32 where mandatory or 1-D, else f16."""
    return {name: W.TensorMeta(tuple(shape), "F32" if W.must_be_f32(name) or len(shape) == 1
                               else "F16")
            for name, shape in W.expected_tree()}


def fake_manifest(tensors):
    return W.Manifest(None, "", "", "test", tensors)


def test_expected_tree_size_and_uniqueness():
    tree = W.expected_tree()
    assert len(tree) == 1334          # 1411 checkpoint keys - 76 bias_masks - 1 mask_token
    assert len({n for n, _ in tree}) == len(tree), "duplicate tensor names"


def test_expected_tree_count_from_structure():
    """The 1334 re-derived part by part: a block has 14 tensors (18 with
    QK-norm); DINO = 7 + 24 blocks; trunk = 3 + 48 QK-norm blocks; camera
    head = 8 + 4 blocks of width 2048; dense head = norm 2 + projects 8 +
    resize 6 + layer_rn 4 + refinenets (3 x 10 + 6) + 2 output convs x 2."""
    tree = W.expected_tree()
    assert len(W.block_tree("x", 1024, False)) == 14
    assert len(W.block_tree("x", 1024, True)) == 18
    count = lambda pre: sum(1 for n, _ in tree if n.startswith(pre))  # noqa: E731
    assert count("aggregator.patch_embed.") == 7 + 24 * 14
    assert count("aggregator.") - count("aggregator.patch_embed.") == 3 + 48 * 18
    assert count("camera_head.") == 8 + 4 * 14
    assert count("dense_head.") == 2 + 8 + 6 + 4 + (3 * 10 + 6) + 4
    assert len(W.trunk_tree(24)) == 3 + 48 * 18
    shapes = dict(tree)
    assert shapes["aggregator.frame_blocks.7.attn.qkv.weight"] == (3072, 1024)
    assert shapes["camera_head.trunk.3.mlp.fc1.weight"] == (8192, 2048)
    assert shapes["aggregator.inter_frame_blocks.23.attn.k_norm.bias"] == (64,)
    assert shapes["dense_head.scratch.layer2_rn.weight"] == (256, 512, 3, 3)
    assert "dense_head.resize_layers.2.weight" not in shapes  # identity level
    assert "dense_head.scratch.refinenet4.resConfUnit1.conv1.weight" not in shapes


@pytest.mark.parametrize("name,want", [
    ("aggregator.frame_blocks.0.ls1.gamma", True), ("aggregator.frame_blocks.0.attn.qkv.bias", True),
    ("aggregator.frame_blocks.0.attn.qkv.weight", False), ("aggregator.frame_blocks.3.norm2.weight", True),
    ("aggregator.inter_frame_blocks.1.attn.q_norm.weight", True),
    ("aggregator.patch_embed.norm.weight", True), ("aggregator.rope_embed.periods", True),
    ("aggregator.camera_token", True), ("aggregator.register_token", True),
    ("aggregator.patch_embed.cls_token", True), ("aggregator.patch_embed.storage_tokens", True),
    ("aggregator.patch_embed.patch_embed.proj.weight", False),
    ("camera_head.camera_branch.2.weight", True), ("camera_head.camera_branch.0.weight", False),
    ("camera_head.token_norm.weight", True), ("dense_head.proj.weight", True),
    ("dense_head.proj_conf.weight", True), ("dense_head.projects.0.weight", False),
    ("dense_head.scratch.refinenet1.out_conv.weight", False),
])
def test_must_be_f32(name, want):
    assert W.must_be_f32(name) is want


def test_manifest_matching_tree_validates():
    W.validate_manifest_tree(fake_manifest(full_fake_tensors()))


def test_manifest_diff_reports_all_mismatch_kinds():
    t = full_fake_tensors()
    del t["aggregator.camera_token"]
    t["aggregator.bogus"] = W.TensorMeta((1,), "F32")
    t["camera_head.trunk_norm.weight"] = W.TensorMeta((7,), "F32")
    # a mandatory-f32 tensor stored as f16 is caught too
    t["aggregator.frame_blocks.0.ls1.gamma"] = W.TensorMeta((1024,), "F16")
    with pytest.raises(W.TreeMismatch) as e:
        W.validate_manifest_tree(fake_manifest(t))
    diff = e.value.diff
    assert "missing from manifest: aggregator.camera_token" in diff
    assert "unexpected in manifest: aggregator.bogus" in diff
    assert "mismatch camera_head.trunk_norm.weight" in diff
    assert "mismatch aggregator.frame_blocks.0.ls1.gamma" in diff
    assert len(diff.splitlines()) == 4, f"no spurious diff lines:\n{diff}"


def test_gemm_weight_may_be_either_dtype():
    t = full_fake_tensors()
    t["aggregator.frame_blocks.0.mlp.fc1.weight"] = W.TensorMeta((4096, 1024), "F32")
    W.validate_manifest_tree(fake_manifest(t))


def tiny_dir(tmp_path, values=None, **over):
    values = values or {"t": np.array([[1, 2], [3, 4]], np.float32)}
    return write_checkpoint(tmp_path, values, over or None)


def test_open_validates_hash_and_contents(tmp_path):
    d = tiny_dir(tmp_path)
    w = W.Weights.open(d, tree=[("t", (2, 2))])
    assert w.tensor("t").shape == (2, 2)
    np.testing.assert_array_equal(w.tensor("t"), [[1, 2], [3, 4]])
    # the manifest's shape corrupted: the contents check fails
    w.manifest.tensors["t"] = W.TensorMeta((4,), "F32")
    with pytest.raises(W.TreeMismatch):
        w.validate_contents()


def test_open_full_tree_refuses_a_partial_checkpoint(tmp_path):
    with pytest.raises(W.TreeMismatch) as e:
        W.Weights.open(tiny_dir(tmp_path))
    assert "unexpected in manifest: t" in e.value.diff
    assert len(e.value.diff.splitlines()) == 1335


def test_open_hash_mismatch(tmp_path):
    d = tiny_dir(tmp_path, model_sha256="00" * 32)
    with pytest.raises(W.HashMismatch) as e:
        W.Weights.open(d, tree=[("t", (2, 2))])
    assert e.value.expected == "00" * 32 and len(e.value.actual) == 64


def test_open_file_holds_other_tensors_than_manifest(tmp_path):
    d = tiny_dir(tmp_path, values={"t": np.zeros((2, 2), np.float32), "u": np.zeros(3, np.float32)})
    m = json.loads((d / "manifest.json").read_text())
    del m["tensors"]["u"]
    (d / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(W.TreeMismatch) as e:
        W.Weights.open(d, tree=[("t", (2, 2))])
    assert "unexpected in file: u" in e.value.diff


def test_open_refuses_unsupported_dtype(tmp_path):
    d = tiny_dir(tmp_path, values={"t": np.zeros((2, 2), np.float64)})
    m = json.loads((d / "manifest.json").read_text())
    m["tensors"]["t"]["dtype"] = "float32"
    (d / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(W.TreeMismatch, match="unsupported dtype F64"):
        W.Weights.open(d, tree=[("t", (2, 2))])


@pytest.mark.parametrize("text,what", [
    ("not json", "manifest parse"),
    ('{"config": null, "checkpoint_sha256": "", "model_sha256": "", "tensors": {}}',
     "conversion_tool_version"),
    ('{"config": null, "checkpoint_sha256": "", "model_sha256": "", "conversion_tool_version": "",'
     ' "tensors": {"t": {"shape": [2], "dtype": "bfloat16"}}}', "bfloat16"),
    ('{"config": null, "checkpoint_sha256": "", "model_sha256": "", "conversion_tool_version": "",'
     ' "tensors": {"t": {"shape": [-2], "dtype": "float16"}}}', "unsigned"),
])
def test_manifest_parse_errors(text, what):
    with pytest.raises(W.ManifestParseError, match=what):
        W.Manifest.parse(text)


def test_missing_files(tmp_path):
    with pytest.raises(W.WeightsIoError):
        W.Weights.open(tmp_path)
    (tmp_path / "manifest.json").write_text(json.dumps(
        {"config": None, "checkpoint_sha256": "", "model_sha256": "", "conversion_tool_version": "",
         "tensors": {}}))
    with pytest.raises(W.WeightsIoError):
        W.Weights.open(tmp_path, tree=[])


# --- the safetensors reader against the library ---------------------------

@pytest.mark.parametrize("seed", range(4))
def test_reader_matches_library(tmp_path, seed):
    rng = np.random.default_rng(seed)
    vals = {}
    kinds = [np.float16, np.float32, np.float64, np.int64, np.int32, np.uint8, np.int8, np.bool_]
    for i in range(int(rng.integers(1, 12))):
        shape = tuple(int(s) for s in rng.integers(0, 5, int(rng.integers(0, 4))))
        dt = kinds[int(rng.integers(len(kinds)))]
        vals[f"t{i}.{seed}"] = np.array(rng.standard_normal(shape) * 50, dtype=dt)
    meta = {"k": "v", "seed": str(seed)}
    p = tmp_path / "x.safetensors"
    stn.save_file(vals, str(p), metadata=meta)
    st = W.SafeTensorsFile(p)
    assert sorted(st.names()) == sorted(vals)
    assert st.metadata == meta
    lib = stn.load_file(str(p))
    for n, a in vals.items():
        got = st.tensor(n)
        assert got.dtype == a.dtype and got.shape == a.shape
        np.testing.assert_array_equal(got, lib[n])
        np.testing.assert_array_equal(got, a)


def raw_file(path, header: dict, data: bytes):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)
    return path


@pytest.mark.parametrize("header,data,what", [
    ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 12, "size"),
    ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
      "b": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 8, "offset"),
    ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 8, "offset"),
    ({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8, "bytes for shape"),
    ({"a": {"dtype": "X9", "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4, "unknown dtype"),
    ({"a": {"dtype": "F32", "shape": [1]}}, b"\0" * 4, "malformed"),
])
def test_reader_refuses_malformed(tmp_path, header, data, what):
    p = raw_file(tmp_path / "bad.safetensors", header, data)
    with pytest.raises(W.SafeTensorsError, match=what):
        W.SafeTensorsFile(p)
    with pytest.raises(Exception):
        stn.load_file(str(p))


def test_reader_refuses_short_and_oversized_headers(tmp_path):
    p = tmp_path / "short.safetensors"
    p.write_bytes(b"\1\2\3")
    with pytest.raises(W.SafeTensorsError, match="too small"):
        W.SafeTensorsFile(p)
    p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(W.SafeTensorsError, match="header length"):
        W.SafeTensorsFile(p)


# --- uploads and the block loader ------------------------------------------

def test_uploads(tmp_path):
    rng = np.random.default_rng(3)
    a32 = (rng.standard_normal((8, 4)) * 3).astype(np.float32)
    a16 = rng.standard_normal((4, 4)).astype(np.float16)
    d = write_checkpoint(tmp_path, {"a32": a32, "a16": a16})
    w = W.Weights.open(d, tree=[("a32", (8, 4)), ("a16", (4, 4))])
    np.testing.assert_array_equal(W.upload_f32(w, "a16", "cpu").numpy(), a16.astype(np.float32))
    got = W.upload_at(w, "a32", torch.float16, "cpu")
    assert got.dtype == torch.float16
    # round to nearest even, as torch's own cast
    np.testing.assert_array_equal(got.numpy(), torch.from_numpy(a32).half().numpy())
    assert W.upload_at(w, "a16", torch.float16, "cpu").numpy().tobytes() == a16.tobytes()
    assert W.upload_at(w, "a16", torch.float32, "cpu").dtype == torch.float32
    with pytest.raises(W.WeightsError):
        W.read_f32(w, "a16")


def test_block_load_splits_qkv(tmp_path):
    from headshot_amd.aggregator import BlockWeights

    tree = W.block_tree("blk", 1024, True)
    vals = synth_values(tree, 7, f32_names={"blk.mlp.fc2.weight"})
    d = write_checkpoint(tmp_path, vals)
    w = W.Weights.open(d, tree=tree)
    b = BlockWeights.load(w, "blk", True, torch.float16, "cpu")
    qkv, qkv_b = vals["blk.attn.qkv.weight"], vals["blk.attn.qkv.bias"]
    for i, (wt, bt) in enumerate(((b.q_w, b.q_b), (b.k_w, b.k_b), (b.v_w, b.v_b))):
        assert wt.dtype == torch.float16 and tuple(wt.shape) == (1024, 1024)
        assert wt.numpy().tobytes() == qkv[i * 1024:(i + 1) * 1024].tobytes()
        assert bt.dtype == torch.float32
        np.testing.assert_array_equal(bt.numpy(), qkv_b[i * 1024:(i + 1) * 1024])
    # the f32-stored fc2 weight comes up rounded to f16
    assert b.fc2_w.dtype == torch.float16
    np.testing.assert_array_equal(b.fc2_w.numpy(),
                                  torch.from_numpy(vals["blk.mlp.fc2.weight"]).half().numpy())
    np.testing.assert_array_equal(b.p.ls2.numpy(), vals["blk.ls2.gamma"])
    np.testing.assert_array_equal(b.p.kn[1].numpy(), vals["blk.attn.k_norm.bias"])
    b32 = BlockWeights.load(w, "blk", True, torch.float32, "cpu")
    np.testing.assert_array_equal(b32.fc1_w.numpy(), vals["blk.mlp.fc1.weight"].astype(np.float32))


# --- reference dumps --------------------------------------------------------

def write_dump(path, tensors, meta):
    stn.save_file(tensors, str(path), metadata={"headshot": json.dumps(meta)})
    return path


def test_dump_reader(tmp_path):
    meta = {"scene": "small", "variant": "f32", "device": "cpu", "n_frames": 2, "width": 64,
            "height": 32, "seed": 42, "shapes": {"x": [2, 3]}}
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    p = write_dump(tmp_path / "dump_small_f32.safetensors",
                   {"x": x, "h": np.zeros(2, np.float16)}, meta)
    d = Dump.open_path(p)
    assert d.meta.scene == "small" and d.meta.n_frames == 2 and d.meta.shapes == {"x": [2, 3]}
    shape, vals = d.tensor("x")
    assert shape == [2, 3]
    np.testing.assert_array_equal(vals, x.ravel())
    with pytest.raises(ValueError, match="must be f32"):
        d.tensor("h")
    assert sorted(d.names()) == ["h", "x"]
    stn.save_file({"x": x}, str(tmp_path / "plain.safetensors"))
    with pytest.raises(ValueError, match="headshot"):
        Dump.open_path(tmp_path / "plain.safetensors")
    with pytest.raises(FileNotFoundError):
        Dump.open_path(tmp_path / "absent.safetensors")


def test_fixtures_dir(monkeypatch, tmp_path):
    monkeypatch.setenv("HEADSHOT_FIXTURES_DIR", str(tmp_path))
    assert fixtures_dir() == tmp_path
    monkeypatch.delenv("HEADSHOT_FIXTURES_DIR")
    assert fixtures_dir().name == "fixtures"
