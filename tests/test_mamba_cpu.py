"""CPU checks of the Mamba mixer pieces: the oracle's conv + SiLU and softplus
against torch's own routines, the oracle's [B,L,D] scan composed into the
mixer against a brute-force fp64 mixer, and the module interface.  No GPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests import _brute


@pytest.mark.parametrize("K", [1, 2, 4, 7])
@pytest.mark.parametrize("with_bias", [True, False])
def test_oracle_conv_silu_matches_torch_conv1d(K, with_bias):
    rng = np.random.default_rng(K)
    x = rng.normal(size=(3, 11, 6))
    w = rng.normal(size=(6, 1, K))
    b = rng.normal(size=6) if with_bias else None
    y = oracle.mamba_conv_silu(x, w, b)
    ref = F.silu(F.conv1d(F.pad(torch.tensor(x).transpose(1, 2), (K - 1, 0)), torch.tensor(w),
                          None if b is None else torch.tensor(b), groups=6)).transpose(1, 2)
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-13, atol=1e-13)


def test_oracle_softplus_matches_torch():
    v = np.concatenate([np.linspace(-40, 40, 401), [19.999, 20.0, 20.001]])
    np.testing.assert_allclose(oracle.softplus(v), F.softplus(torch.tensor(v)).numpy(),
                               rtol=1e-14, atol=1e-300)


def _mixer_params(rng, d_model, d_inner, d_state, d_conv, dt_rank):
    t = lambda *s, scale=1.0: torch.tensor(rng.normal(size=s) * scale)
    return {
        "in_proj.weight": t(2 * d_inner, d_model, scale=d_model ** -0.5),
        "conv1d.weight": t(d_inner, 1, d_conv, scale=0.5),
        "conv1d.bias": t(d_inner, scale=0.1),
        "x_proj.weight": t(dt_rank + 2 * d_state, d_inner, scale=d_inner ** -0.5),
        "dt_proj.weight": t(d_inner, dt_rank, scale=dt_rank ** -0.5),
        "dt_proj.bias": torch.tensor(rng.uniform(-5, -2, d_inner)),
        "A_log": torch.log(torch.arange(1, d_state + 1, dtype=torch.float64).repeat(d_inner, 1)),
        "out_proj.weight": t(d_model, d_inner, scale=d_inner ** -0.5),
    }


def test_oracle_mixer_pieces_compose_to_the_brute_mixer():
    """in_proj / x_proj / dt_proj / out_proj as numpy GEMMs around the oracle's
    conv + SiLU and [B,L,D] scan reproduce the brute-force fp64 mixer."""
    rng = np.random.default_rng(1)
    d_model, d_inner, d_state, d_conv, dt_rank = 8, 12, 5, 4, 2
    p = _mixer_params(rng, d_model, d_inner, d_state, d_conv, dt_rank)
    u = torch.tensor(rng.normal(size=(2, 17, d_model)))
    ref = _brute.mamba_mixer(u, p, d_conv, dt_rank, d_state).numpy()
    n = {k: v.numpy() for k, v in p.items()}
    xz = u.numpy() @ n["in_proj.weight"].T
    x, z = xz[..., :d_inner], xz[..., d_inner:]
    xc = oracle.mamba_conv_silu(x, n["conv1d.weight"], n["conv1d.bias"])
    proj = xc @ n["x_proj.weight"].T
    dt_pre = proj[..., :dt_rank] @ n["dt_proj.weight"].T
    Bg, Cg = proj[..., dt_rank:dt_rank + d_state], proj[..., dt_rank + d_state:]
    y = oracle.selective_forward_bld(xc, dt_pre, -np.exp(n["A_log"]), Bg, Cg, gate=z,
                                     dt_bias=n["dt_proj.bias"])
    out = y @ n["out_proj.weight"].T
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_mixer_module_interface():
    from ossm_amd.mamba import MambaMixer

    m = MambaMixer(16, d_state=8, d_conv=4, expand=2)
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    # the reference _MambaMixer's parameters (mambarec.py:92-133), dt_rank = ceil(16/16) = 1
    assert shapes == {"in_proj.weight": (64, 16), "conv1d.weight": (32, 1, 4),
                      "conv1d.bias": (32,), "x_proj.weight": (17, 32), "dt_proj.weight": (32, 1),
                      "dt_proj.bias": (32,), "out_proj.weight": (16, 32), "A_log": (32, 8)}
    # dt_proj.bias is softplus^-1 of dt in [dt_min, dt_max] (mambarec.py:120-124)
    dt = F.softplus(m.dt_proj.bias.detach())
    assert float(dt.min()) >= 1e-3 * (1 - 1e-5) and float(dt.max()) <= 0.1 * (1 + 1e-5)
    torch.testing.assert_close(-torch.exp(m.A_log.detach())[0], -torch.arange(1.0, 9.0))
    with pytest.raises(ValueError, match="shape \\(batch, length, channels\\)"):
        m(torch.zeros(2, 16))
    with pytest.raises(RuntimeError, match="GPU only"):
        m(torch.zeros(1, 3, 16))
    assert m(torch.zeros(1, 0, 16)).shape == (1, 0, 16)


def test_mixer_entries_reject_what_the_kernels_cannot_read():
    from ossm_amd.mamba import mamba_conv_silu, selective_scan_mamba

    x = torch.zeros(1, 4, 8)
    with pytest.raises(RuntimeError, match="float32 GPU tensor"):
        mamba_conv_silu(x, torch.zeros(8, 1, 4))
    with pytest.raises(RuntimeError, match="float32 GPU tensor"):
        selective_scan_mamba(x, x, torch.zeros(8, 2), torch.zeros(1, 4, 2), torch.zeros(1, 4, 2))
