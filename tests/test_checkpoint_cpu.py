"""Checkpoint loader (mace_ictc.checkpoints.load_checkpoint) on the CPU.

A checkpoint written in the reference's layout (e3trans_* state dicts,
model_hyperparameters, E0 keys/values; mace_ictc/training/train_loop.py:
1728-1850) reloads into a model whose parameter names, shapes and values
equal the saved ones, with the architecture read back from the metadata and
weight shapes: the float64 oracle gives the reloaded model the same energies
and forces as the original.  Also: EMA/SWA/raw selection, the reference's
legacy defaults (polynomial p = 6, sqrt(num_basis) radial norm), and the
refusals (other backbones, options outside the baseline, pickled objects).
"""
import argparse
import math

import pytest
import torch

import model_oracle as mo
from model_helpers import build_graph, fcc_cells


def _model(**kw):
    from mace_ictc.hp.model import PureCartesianICTDFix
    torch.manual_seed(kw.pop("seed", 0))
    args = dict(channels=8, lmax=2, atomic_numbers=(1, 6, 8), cutoff=4.5, avg_num_neighbors=30.0)
    args.update(kw)
    return PureCartesianICTDFix(**args)


def _ckpt(model, **extra):
    hp = {"lmax": model.lmax, "channel_in": model.channels, "num_interaction": model.num_interaction,
          "function_type": "bessel", "number_of_basis": model.number_of_basis,
          "avg_num_neighbors": model.avg_num_neighbors, "ictd_fix_edge_lmax": model.ictd_fix_edge_lmax,
          "polynomial_cutoff_p": model.polynomial_cutoff_p, "radial_sqrt_num_basis": model.radial_sqrt_num_basis,
          "ictd_fix_route": "baseline", "dtype": "float32"}
    ck = {"e3trans_state_dict": model.state_dict(), "model_hyperparameters": hp,
          "tensor_product_mode": "pure-cartesian-ictd-fix", "max_radius": model.max_radius,
          "atomic_energy_keys": torch.tensor(model.atomic_numbers),
          "atomic_energy_values": torch.tensor([-0.5, -37.8, -75.0][:model.num_elements], dtype=torch.float64)}
    ck.update(extra)
    return ck


def _energies(model):
    pos, Z, batch, cell = fcc_cells(2, 0.1, 0.3, 3, model.num_elements, atomic_numbers=model.atomic_numbers)
    src, dst, sh = build_graph(pos, batch, cell, model.max_radius)
    return mo.energy_and_forces(model.state_dict(), mo.config_of(model), pos, Z, batch, src, dst, sh, cell, 1)


def test_reload_reproduces_parameters_and_energies(tmp_path):
    from mace_ictc.checkpoints import load_checkpoint
    model = _model(edge_lmax=3, correlation=2)
    path = tmp_path / "model.pth"
    torch.save(_ckpt(model), path)
    pot = load_checkpoint(str(path), ["H", "C", "O"])
    got = pot.model
    assert set(got.state_dict()) == set(model.state_dict())
    for k, v in model.state_dict().items():
        assert torch.equal(got.state_dict()[k], v), k
    assert got.ictd_fix_edge_lmax == 3 and got.products[0].symmetric_contractions.correlation == 2
    assert got.avg_num_neighbors == 30.0 and got.max_radius == 4.5
    E0, F0, _ = _energies(model)
    E1, F1, _ = _energies(got)
    assert torch.allclose(E1, E0, rtol=0, atol=1e-12) and torch.allclose(F1, F0, rtol=0, atol=1e-12)
    assert pot.element_types == ["H", "C", "O"]
    assert torch.equal(pot.wrapper.atomic_energy_keys, torch.tensor([1, 6, 8]))
    assert all(not p.requires_grad for p in got.parameters())


def test_state_source_selection(tmp_path):
    from mace_ictc.checkpoints import get_checkpoint_e3_state_dict, load_checkpoint
    model, ema, swa = _model(seed=1), _model(seed=2), _model(seed=3)
    ck = _ckpt(model, e3trans_ema_state_dict=ema.state_dict(), e3trans_swa_state_dict=swa.state_dict())
    assert get_checkpoint_e3_state_dict(ck)[1] == "ema"              # EMA preferred by default
    assert get_checkpoint_e3_state_dict(ck, prefer_ema=False)[1] == "raw"
    ck["default_state_source"] = "swa"
    assert get_checkpoint_e3_state_dict(ck)[1] == "swa"
    path = tmp_path / "m.pth"
    torch.save(ck, path)
    got = load_checkpoint(str(path), ["H", "C", "O"]).model
    w = "node_embedding.weight"
    assert torch.equal(got.state_dict()[w], swa.state_dict()[w])
    with pytest.raises(KeyError):
        get_checkpoint_e3_state_dict({"model_hyperparameters": {}})


def test_legacy_defaults_sqrt_norm_and_cutoff_order(tmp_path):
    """Without radial_sqrt_num_basis / polynomial_cutoff_p in the metadata the reference rebuilds with
    sqrt(num_basis) on and p = 6 (loader.py:443-454); the oracle energies follow the rebuilt radial basis."""
    from mace_ictc.checkpoints import load_checkpoint
    model = _model(polynomial_cutoff_p=6, radial_sqrt_num_basis=True)
    ck = _ckpt(model)
    del ck["model_hyperparameters"]["radial_sqrt_num_basis"], ck["model_hyperparameters"]["polynomial_cutoff_p"]
    path = tmp_path / "legacy.pth"
    torch.save(ck, path)
    got = load_checkpoint(str(path), ["H", "C", "O"]).model
    assert got.radial_sqrt_num_basis and got.polynomial_cutoff_p == 6
    assert got.radial_basis_scale == pytest.approx(math.sqrt(8))
    E0, F0, _ = _energies(model)
    E1, F1, _ = _energies(got)
    assert torch.allclose(E1, E0, rtol=0, atol=1e-12) and torch.allclose(F1, F0, rtol=0, atol=1e-12)
    # the norm changes the energies (the check above is not vacuous)
    plain = _model(polynomial_cutoff_p=6)
    plain.load_state_dict(model.state_dict())
    E2, _, _ = _energies(plain)
    assert not torch.allclose(E2, E0, rtol=0, atol=1e-6)


def test_refusals(tmp_path):
    from mace_ictc.checkpoints import load_checkpoint
    model = _model()
    cases = {
        "mode": _ckpt(model, tensor_product_mode="spherical"),
        "route": _ckpt(model, ictd_fix_route="fusion"),
        "long_range": _ckpt(model, model_hyperparameters=dict(_ckpt(model)["model_hyperparameters"],
                                                              long_range_mode="reciprocal-spectral")),
        "pickle": _ckpt(model, config=argparse.Namespace(lmax=2)),
    }
    for name, ck in cases.items():
        path = tmp_path / f"{name}.pth"
        torch.save(ck, path)
        with pytest.raises(ValueError):
            load_checkpoint(str(path), ["H", "C", "O"])
    ck = _ckpt(model)
    del ck["model_hyperparameters"]["avg_num_neighbors"]
    path = tmp_path / "noavg.pth"
    torch.save(ck, path)
    with pytest.warns(RuntimeWarning, match="avg_num_neighbors"):
        got = load_checkpoint(str(path), ["H", "C", "O"]).model
    assert got.avg_num_neighbors == 14.38


def test_missing_function_type_resolves_to_gaussian(tmp_path):
    """Reference mace_ictc/checkpoints/loader.py:156 reads a missing function_type as 'gaussian'; a Gaussian
    radial basis is not built here, so such a checkpoint must be refused rather than loaded as Bessel."""
    from mace_ictc.checkpoints import load_checkpoint
    model = _model()
    ck = _ckpt(model)
    del ck["model_hyperparameters"]["function_type"]
    path = tmp_path / "noft.pth"
    torch.save(ck, path)
    with pytest.raises(ValueError, match="gaussian"):
        load_checkpoint(str(path), ["H", "C", "O"])
    ck = _ckpt(model, function_type="bessel")
    del ck["model_hyperparameters"]["function_type"]
    torch.save(ck, path)
    assert load_checkpoint(str(path), ["H", "C", "O"]).model.number_of_basis == model.number_of_basis
