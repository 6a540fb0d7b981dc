"""The offline float quantiser (idempotent_llm_amd.prepare, the contract of
the reference's src/detllm/prepare.py):

* the fitting helpers against vectors the reference's own helpers wrote
  (tests/golden/prepare_helpers.npz, make_prepare_golden.py) — exact;
* the whole quantisation of a small random Qwen3 float model with fixed
  calibration ids against the artifact the reference's prepare() wrote for
  the same model and ids (tests/golden/prepare_artifact.json,
  make_prepare_artifact.py): every tensor byte-identical (SHA-256, and the
  values of the int64 scale tensors) and an equal config, with and without
  smoothing; a planted change to the smoothing's median normalisation or to
  its clamp fails that comparison;
* the artifact has the runtime schema (names, dtypes, shapes and config keys
  of the random-init generator), loads in the integer oracle, and the
  integer model's logits track the float model's."""

import contextlib
import json
import os

import numpy as np
import pytest
import torch

from artifact_record import describe, differences
from floatmodel import small_float_model
from idempotent_llm_amd import prepare as P

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def G():
    return dict(np.load(os.path.join(HERE, "golden", "prepare_helpers.npz")))


def test_scalar_and_vector_fits(G):
    s = G["fit_s"]
    got = np.array([P.fit_dyadic_float(float(v)) for v in s], dtype=np.int64)
    assert np.array_equal(got[:, 0], G["fit_m"]) and np.array_equal(got[:, 1], G["fit_k"])
    got14 = np.array([P.fit_dyadic_float(float(v), 14) for v in s[:500]], dtype=np.int64)
    assert np.array_equal(got14[:, 0], G["fit14_m"]) and np.array_equal(got14[:, 1], G["fit14_k"])
    m, k = P.fit_dyadic_float_vec(torch.from_numpy(s))
    assert np.array_equal(m.numpy(), G["vec_m"]) and np.array_equal(k.numpy(), G["vec_k"])
    # what the fit means: m in [2^15, 2^16) and m / 2^k within half a unit of s
    assert (got[:, 0] >= 1 << 15).all() and (got[:, 0] < 1 << 16).all()
    err = np.abs(got[:, 0] * np.exp2(-got[:, 1].astype(np.float64)) - s)
    assert (err <= 0.5 * np.exp2(-got[:, 1].astype(np.float64)) * (1 + 1e-12)).all()


@pytest.mark.parametrize("bits", [8, 16])
def test_weight_per_channel(G, bits):
    W = torch.from_numpy(G["w"]).float()
    q, m, k = P.quant_weight_per_channel(W, weight_bits=bits)
    assert q.dtype == (torch.int8 if bits == 8 else torch.int16)
    assert np.array_equal(q.numpy(), G[f"w{bits}_q"])
    assert np.array_equal(m.numpy(), G[f"w{bits}_m"]) and k == int(G[f"w{bits}_k"])


def test_embedding_and_gamma(G):
    e8, em, ek = P.quant_embedding_per_row(torch.from_numpy(G["e"]))
    assert np.array_equal(e8.numpy(), G["e8"])
    assert np.array_equal(em.numpy(), G["em"]) and np.array_equal(ek.numpy(), G["ek"])
    gm, gk = P.fit_gamma_dyadic(torch.from_numpy(G["gamma"]))
    assert np.array_equal(gm.numpy(), G["gamma_m"]) and gk == int(G["gamma_k"])


@pytest.fixture(scope="module")
def ref_artifact():
    with open(os.path.join(HERE, "golden", "prepare_artifact.json")) as f:
        return json.load(f)


@contextlib.contextmanager
def _one_thread():
    # the reference's artifact was written with one CPU thread: the float
    # calibration pass then sums in the same order here
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        yield
    finally:
        torch.set_num_threads(n)


def _quantise(out_dir, rec):
    calib = np.random.default_rng(5).integers(0, 1000, (4, 64), dtype=np.int64)
    with _one_thread():
        P.prepare(out_dir, small_float_model(seed=0, **rec["model_options"]), calib,
                  device="cpu", model_id="test-small-qwen3", **rec["options"])
    return describe(out_dir)


@pytest.mark.parametrize("variant", ["default", "no_smoothing_qk_alpha_0p5",
                                     "outlier_channels"])
def test_artifact_identical_to_the_reference(ref_artifact, variant, tmp_path):
    """prepare() writes the reference's artifact bit for bit (prepare.py:
    120-434: calibration maxima, activation and QK smoothing, static K/V
    scales, every fit)."""
    want = ref_artifact["variants"][variant]
    got = _quantise(str(tmp_path), want)
    assert len(got["tensors"]) == len(want["tensors"]) == 61
    assert differences(got, want) == []


@pytest.mark.parametrize("plant", ["mean_normalisation", "clamp_32", "clamp_128"])
def test_planted_smoothing_change_fails(ref_artifact, plant, tmp_path, monkeypatch):
    """A plausible slip in the smoothing formulas (mean instead of median
    normalisation, another clamp bound) changes the artifact: the comparison
    above catches it (the outlier-channel model drives factors past the
    clamp at every smoothing site)."""
    if plant == "mean_normalisation":
        monkeypatch.setattr(P, "_relative", lambda s: s / s.mean())
    else:
        monkeypatch.setattr(P, "SMOOTH_CLAMP", float(plant.split("_")[1]))
    want = ref_artifact["variants"]["outlier_channels"]
    diff = differences(_quantise(str(tmp_path), want), want)
    sites = {d.rsplit(".", 1)[-1] for d in diff}
    assert {"as_m", "ms_m", "ds_m", "os_m"} <= sites, diff
    if plant != "mean_normalisation":          # QK smoothing shares the clamp
        assert "qs_m" in sites, diff


@pytest.fixture(scope="module")
def prepared(tmp_path_factory):
    model = small_float_model()
    rng = np.random.default_rng(5)
    calib = rng.integers(0, 1000, (4, 64), dtype=np.int64)
    d = str(tmp_path_factory.mktemp("prepared"))
    P.prepare(d, model, calib, device="cpu", model_id="test-small-qwen3")
    return model, d


def test_artifact_schema_matches_the_runtime(prepared):
    from safetensors.numpy import load_file
    from idempotent_llm_amd import artifact as art
    _, d = prepared
    t = load_file(os.path.join(d, "model.safetensors"))
    with open(os.path.join(d, "config.json")) as f:
        cfg = json.load(f)
    ref_t, ref_cfg = art.make_artifact_tensors(art.TINY, seed=1)
    assert set(t) == set(ref_t)
    for name, v in ref_t.items():
        assert t[name].dtype == v.dtype, name
        assert t[name].shape == v.shape, name
    for key in ref_cfg:
        assert key in cfg, key
    assert set(cfg["layers"][0]) >= set(ref_cfg["layers"][0])
    for name, v in t.items():
        assert np.issubdtype(v.dtype, np.integer), name
    # the RoPE tables are the runtime's own (pinned against the reference's
    # build_rope_tables digest in the golden tests)
    cos_t, _ = art.rope_tables(128, 1024, 1e6)
    assert np.array_equal(t["rope.cos"], cos_t)


def test_integer_model_tracks_the_float_model(prepared):
    """Prefill logits of the quantised model (integer oracle) against the float
    model: per position, logits * head_m correlate with the float logits."""
    from oracle.model import IntQwen3Oracle
    model, d = prepared
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 1000, (1, 24), dtype=np.int64)
    orc = IntQwen3Oracle(d)
    logits = orc.forward(ids, np.arange(24, dtype=np.int64)[None])[0]
    with torch.no_grad():
        ref = model(torch.from_numpy(ids)).logits[0].double().numpy()
    from safetensors.numpy import load_file
    head_m = load_file(os.path.join(d, "model.safetensors"))["head.m"].astype(np.float64)
    approx = logits[0].astype(np.float64) * head_m[None, :]
    corr = [np.corrcoef(approx[t], ref[t])[0, 1] for t in range(24)]
    assert min(corr) > 0.98, corr
    agree = np.mean(approx.argmax(-1) == ref.argmax(-1))
    assert agree >= 0.6, agree
