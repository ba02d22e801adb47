"""Real-checkpoint parity (crates/headshot-server/tests/parity.rs), against
locally generated fixtures: a converted checkpoint (``manifest.json`` +
``model.safetensors``, from the reference's tools/convert_weights.py) in
``fixtures_dir()`` and reference activation dumps (tools/dump_reference.py)
under its ``dumps/``. Fixtures derive from a gated checkpoint and are never
committed; without them every test here is skipped, as the reference's own
parity suite is ``#[ignore]``d.

The trunk runs from the dump's own DINO output (``dino.tokens``): this
library's path starts at the trunk's token assembly. Gates are the
reference's (parity.rs:66-84): the all-f32 trunk against the f32 dump with
F32_DEEP; the f16 trunk against the bf16 dump with F16_TRUNK, widened per
tap to twice the reference's own bf16-vs-f32 drift where that is larger
(tests/parity.rs:74-121).
"""
import numpy as np
import pytest
import torch

from headshot_amd.parity import Dump, Gate, compare, fixtures_dir

SCENES = ("small", "realistic")


def have_weights():
    return (fixtures_dir() / "manifest.json").is_file() and (fixtures_dir() / "model.safetensors").is_file()


def have_dump(scene, variant):
    return (fixtures_dir() / "dumps" / f"dump_{scene}_{variant}.safetensors").is_file()


needs_weights = pytest.mark.skipif(not have_weights(),
                                   reason="needs locally converted weights in fixtures_dir()")


@needs_weights
def test_parity_weights_load_and_validate():
    """tests/parity.rs:21-34: the converted checkpoint loads, matches the
    expected tree and the manifest, and its checksum round-trips."""
    from headshot_amd.weights import Weights

    w = Weights.open(fixtures_dir())
    assert len(w.manifest.tensors) == 1334
    periods = w.tensor("aggregator.rope_embed.periods")
    assert periods.shape == (16,)
    assert np.all(np.isfinite(periods)) and np.all(periods > 0)


@pytest.mark.parametrize("scene", SCENES)
@pytest.mark.parametrize("variant", ["bf16", "f32"])
def test_parity_dumps_are_consistent(scene, variant):
    """tests/parity.rs:36-67."""
    if not have_dump(scene, variant):
        pytest.skip("needs locally generated reference dumps")
    dump = Dump.open(scene, variant)
    assert dump.meta.scene == scene and dump.meta.variant == variant
    shape, images = dump.tensor("images")
    assert shape == [dump.meta.n_frames, 3, dump.meta.height, dump.meta.width]
    assert np.all((images >= 0.0) & (images <= 1.0))
    for name, want in dump.meta.shapes.items():
        assert dump.tensor(name)[0] == want, f"{scene}/{variant}: {name}"


@pytest.mark.gpu
@pytest.mark.parametrize("scene", SCENES)
@pytest.mark.parametrize("precision", ["f32", "f16"])
def test_parity_trunk(ctx, scene, precision):
    """The trunk part of trunk_parity (tests/parity.rs:69-160): every
    trunk.frame.NN, trunk.inter.NN and cache.NN tap against the dump."""
    variant = "f32" if precision == "f32" else "bf16"
    if not (have_weights() and have_dump(scene, variant) and have_dump(scene, "f32")):
        pytest.skip("needs locally converted weights and reference dumps")
    from headshot_amd.trunk import Trunk
    from headshot_amd.weights import Weights

    dt = torch.float32 if precision == "f32" else torch.float16
    trunk = Trunk.load(Weights.open(fixtures_dir()), dt, "cuda:0")
    dump = Dump.open(scene, variant)
    other = Dump.open(scene, "f32") if precision == "f16" else None
    n = dump.meta.n_frames
    h_p, w_p = dump.meta.height // 16, dump.meta.width // 16
    _, tokens = dump.tensor("dino.tokens")
    base = Gate.F32_DEEP if precision == "f32" else Gate.F16_TRUNK
    failures = []

    def tap(name, t):
        if name not in dump.meta.shapes:
            return
        torch.cuda.synchronize()
        ours = t.float().cpu().numpy().ravel()
        ref_shape, ref = dump.tensor(name)
        assert ours.size == int(np.prod(ref_shape)), f"{name}: element count vs dump {ref_shape}"
        m = compare(ours, ref)
        gate = base
        if other is not None:
            _, f32_ref = other.tensor(name)
            drift = 1.0 - compare(ref, f32_ref).cosine_sim
            gate = Gate(gate.rel_max, 1.0 - max(1.0 - gate.min_cosine, 2.0 * drift))
        print(f"{name:>16}: rel_max {m.rel_max_err():.3e}  cosine 1-{1.0 - m.cosine_sim:.3e}")
        try:
            gate.check(name, m)
        except AssertionError as e:
            failures.append(str(e))

    caches = trunk.forward(ctx, torch.from_numpy(tokens).to("cuda:0").reshape(n * h_p * w_p, 1024),
                           n, h_p, w_p, tap=tap)
    assert len(caches) == 4
    assert not failures, "parity gate failures:\n" + "\n".join(failures)
