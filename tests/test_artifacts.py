"""Artifact loader and read-rotation folding (CPU): the reference's checks and the fold's algebra.

Reference behaviour: deployment/sglang/srt/mem_cache/rolaq_mla.py:16-71 and the
rotation validator mla_quant/quantizer.py:145-152. The reference ships no
artifact, so these tests write artifacts in its format and pin the loader
against every rule it enforces, and the fold against closed forms (identity,
permutation) and the absorbed-attention identity it exists for.
"""

import json

import pytest
import torch

from mla_kv_quant_amd import artifacts, synth
from oracle import codec

MODEL = {"model_type": "deepseek_v2", "num_hidden_layers": 3, "kv_lora_rank": 256, "qk_rope_head_dim": 32}


def make_artifact(tmp_path, name="art", width=256, layers=3, params=None):
    rots = {i: synth.make_rotation(width, 100 + i) for i in range(layers)}
    params = params or {i: (0.75 + 0.1 * i, codec.signal_gain(0.75 + 0.1 * i)) for i in range(layers)}
    model = dict(MODEL, num_hidden_layers=layers, kv_lora_rank=width)
    root = tmp_path / name
    artifacts.write_artifact(root, rots, params, model)
    artifacts.open_artifact.cache_clear()
    return root, rots, params


def edit_manifest(root, fn):
    m = json.loads((root / "manifest.json").read_text())
    fn(m)
    (root / "manifest.json").write_text(json.dumps(m))
    artifacts.open_artifact.cache_clear()


def test_quantizers_round_trip_and_no_artifact(tmp_path):
    root, rots, params = make_artifact(tmp_path)
    got = artifacts.load_layer_quantizers(str(root), str(root), 128, 256, [2, 0])
    assert got == [params[2], params[0]]
    assert artifacts.load_layer_quantizers(None, None, 128, 256, [0, 1]) == [None, None]
    assert artifacts.load_layer_quantizers("", "x", 128, 256, [5]) == [None]
    for i, r in rots.items():
        assert torch.equal(artifacts.load_rotation(root, i, 256), r)


@pytest.mark.parametrize("key,value", [("recipe", "v1"), ("family", "uniform"), ("components", ["nope", "pe"]),
                                       ("group_size", 64)])
def test_manifest_schema_is_enforced(tmp_path, key, value):
    root, _, _ = make_artifact(tmp_path)
    edit_manifest(root, lambda m: m.__setitem__(key, value))
    with pytest.raises(ValueError):
        artifacts.load_layer_quantizers(str(root), str(root), 128, 256, [0])


def test_every_layer_file_and_hash_is_checked(tmp_path):
    root, _, _ = make_artifact(tmp_path, "missing")
    edit_manifest(root, lambda m: m["layers"].pop("1"))
    with pytest.raises(ValueError, match="one record per decoder layer"):
        artifacts.load_layer_quantizers(str(root), str(root), 128, 256, [0])
    root, _, _ = make_artifact(tmp_path, "renamed")
    edit_manifest(root, lambda m: m["layers"]["0"].__setitem__("file", "layer_00.pt"))
    with pytest.raises(ValueError, match="file name"):
        artifacts.load_layer_quantizers(str(root), str(root), 128, 256, [0])
    root, _, _ = make_artifact(tmp_path, "tampered")
    torch.save(synth.make_rotation(256, 999), root / "layer_1.pt")  # same shape, other bytes
    artifacts.open_artifact.cache_clear()
    with pytest.raises(ValueError, match="SHA-256"):
        artifacts.load_layer_quantizers(str(root), str(root), 128, 256, [0])


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), 0.0, -0.5])
def test_quantizer_parameters_must_be_finite_positive(tmp_path, bad):
    root, _, _ = make_artifact(tmp_path)
    edit_manifest(root, lambda m: m["layers"]["2"].__setitem__("param1", bad))
    with pytest.raises(ValueError, match="finite and positive"):
        artifacts.load_layer_quantizers(str(root), str(root), 128, 256, [0])


def test_artifact_must_match_cache_and_rotation_source(tmp_path):
    root, _, _ = make_artifact(tmp_path, "a")
    other, _, _ = make_artifact(tmp_path, "b")
    with pytest.raises(ValueError, match="one artifact"):
        artifacts.load_layer_quantizers(str(root), str(other), 128, 256, [0])
    with pytest.raises(ValueError, match="latent width"):
        artifacts.load_layer_quantizers(str(root), str(root), 128, 512, [0])
    with pytest.raises(ValueError, match="latent width"):
        artifacts.load_layer_quantizers(str(root), str(root), 64, 256, [0])


def test_rotation_checks(tmp_path):
    d = tmp_path / "rot"
    d.mkdir()
    r = synth.make_rotation(128, 5)
    cases = {
        0: r.double(),                       # not FP32
        1: r[:, :64].contiguous(),           # not square
        2: r * 1.001,                        # not orthogonal
        3: r.clone().index_put_((torch.tensor([0]), torch.tensor([0])), torch.tensor(float("nan"))),
    }
    for i, t in cases.items():
        torch.save(t, d / f"layer_{i}.pt")
        with pytest.raises(ValueError):
            artifacts.load_rotation(d, i, 128)
    torch.save(r, d / "layer_9.pt")
    assert torch.equal(artifacts.load_rotation(d, 9, 128), r)
    with pytest.raises(ValueError):
        artifacts.load_rotation(d, 9, 256)  # width mismatch


def test_fold_read_rotation_closed_forms(tmp_path):
    d = tmp_path / "fold"
    d.mkdir()
    width, rows = 128, 48
    w = synth.make_normal((rows, width), 3)
    torch.save(torch.eye(width), d / "layer_0.pt")
    assert torch.equal(artifacts.fold_read_rotation(w, 0, d), w)
    perm = torch.randperm(width, generator=torch.Generator().manual_seed(1))
    p = torch.eye(width)[:, perm]              # W @ P permutes W's columns exactly
    torch.save(p, d / "layer_1.pt")
    assert torch.equal(artifacts.fold_read_rotation(w, 1, d), w[:, perm])
    with pytest.raises(ValueError):
        artifacts.fold_read_rotation(w.float(), 1, d)
    with pytest.raises(ValueError):
        artifacts.fold_read_rotation(w[:, :64].contiguous(), 1, d)


def test_fold_read_rotation_absorbs_the_cache_rotation(tmp_path):
    """q . (W_k R) applied to the rotated latent c R equals q . W_k c up to bf16 rounding,
    which is why the absorbed readers can work in the rotated frame."""
    d = tmp_path / "absorb"
    d.mkdir()
    width = 256
    r = synth.make_rotation(width, 11)
    torch.save(r, d / "layer_0.pt")
    wk = synth.make_normal((64, width), 4, std=0.05)
    folded = artifacts.fold_read_rotation(wk, 0, d).float()
    # the fold is W_b @ R_eff with R_eff = fp32(bf16(R)), rounded once to bf16
    r_eff = r.to(torch.bfloat16).float()
    exact = wk.double() @ r_eff.double()
    assert (folded.double() - exact).abs().max() <= 2 ** -8 * exact.abs().max()
    c = synth.make_latent(32, width, 3, seed=6).float()
    rotated = c @ r_eff                          # what the writer stores (before quantization)
    lhs = rotated.double() @ folded.double().T   # absorbed score against the rotated latent
    rhs = c.double() @ wk.double().T             # un-rotated reference
    assert torch.allclose(lhs, rhs, rtol=0, atol=0.03 * rhs.abs().max().item())


def test_gpu_quantizer_checks_before_any_launch(tmp_path):
    """The GPU inference quantizer's contract (mla_quant/quantizer.py:218-316):
    construction checks, the ValueError cases of quantize_layer and the config
    check -- all raised on the host before any kernel would run."""
    from types import SimpleNamespace

    from mla_kv_quant_amd.qdq import LearnedRotationQuantizer

    root, rots, params = make_artifact(tmp_path, layers=2)
    q = LearnedRotationQuantizer(root)
    assert q.width == 256 and set(q.rotations) == {0, 1} and q.params[1] == params[1]
    x = torch.zeros(1, 4, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="nope only"):
        q.quantize_layer(x, 0, "rope")
    with pytest.raises(ValueError, match="shape or dtype"):
        q.quantize_layer(torch.zeros(1, 4, 128, dtype=torch.bfloat16), 0, "nope")
    with pytest.raises(ValueError, match="shape or dtype"):
        q.quantize_layer(torch.zeros(1, 4, 256, dtype=torch.int32), 0, "nope")
    with pytest.raises(ValueError, match="missing learned rotation"):
        q.quantize_layer(x, 5, "nope")
    assert q.call_count == 0
    q.validate_config(SimpleNamespace(**dict(MODEL, num_hidden_layers=2)))
    with pytest.raises(ValueError, match="kv_lora_rank"):
        q.validate_config(SimpleNamespace(**dict(MODEL, num_hidden_layers=2, kv_lora_rank=512)))
    # a tampered rotation file fails its SHA-256 at construction
    torch.save(torch.eye(256), root / "layer_1.pt")
    with pytest.raises(ValueError, match="SHA-256"):
        LearnedRotationQuantizer(root)
