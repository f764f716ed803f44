"""Pins the absorbed-MLA oracle with the reference's own known-answer test.

tests/test_mla_absorbed.py:115-222 of the reference draws its inputs from
numpy default_rng(34) in a fixed order, so they are reproducible without MLX.
Its expected value is the expanded (non-absorbed) attention; here that is
computed in float64 independently of the absorbed formula, and the oracle's
absorbed and key-tiled forms must match it within the reference's
tolerances (2e-5 dense, 3e-5 tiled).
"""
import numpy as np
import pytest

from oracle import bf16 as obf
from oracle import mla


def reference_inputs():
    rng = np.random.default_rng(34)
    B, heads, length, offset = 1, 3, 5, 3
    total = offset + length
    dn, dr, dv, latent = 4, 2, 5, 6
    hidden = 17
    q_nope = rng.standard_normal((B, heads, length, dn)).astype(np.float32)
    q_rope = rng.standard_normal((B, heads, length, dr)).astype(np.float32)
    c_all = rng.standard_normal((B, total, latent)).astype(np.float32)
    k_rope = rng.standard_normal((B, total, dr)).astype(np.float32)
    kv_b = rng.standard_normal((heads * (dn + dv), latent)).astype(np.float32)
    o_proj = rng.standard_normal((hidden, heads * dv)).astype(np.float32)
    return dict(q_nope=q_nope, q_rope=q_rope, c_all=c_all, k_rope=k_rope, kv_b=kv_b,
                o_proj=o_proj, offset=offset, dn=dn, dv=dv)


def test_absorbed_and_tiled_match_expanded_reference_test():
    r = reference_inputs()
    lat = np.concatenate([r["c_all"], r["k_rope"]], axis=-1)
    exp = mla.project(mla.expanded(r["q_nope"], r["q_rope"], r["c_all"], r["k_rope"], r["kv_b"],
                                   r["dn"], r["dv"], offset=r["offset"]), r["o_proj"])
    dense, _ = mla.absorbed(r["q_nope"], r["q_rope"], lat, r["kv_b"], r["dn"], r["dv"],
                            offset=r["offset"])
    tiled, _ = mla.absorbed(r["q_nope"], r["q_rope"], lat, r["kv_b"], r["dn"], r["dv"],
                            offset=r["offset"], key_tile_size=3)
    np.testing.assert_allclose(mla.project(dense, r["o_proj"]), exp, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(mla.project(tiled, r["o_proj"]), exp, atol=3e-5, rtol=3e-5)


def test_mistakes_in_the_absorption_are_caught():
    # Planted mistakes in a CPU copy of the inputs must break the identity.
    r = reference_inputs()
    lat = np.concatenate([r["c_all"], r["k_rope"]], axis=-1)
    exp = mla.expanded(r["q_nope"], r["q_rope"], r["c_all"], r["k_rope"], r["kv_b"],
                       r["dn"], r["dv"], offset=r["offset"])
    wrong_scale, _ = mla.absorbed(r["q_nope"], r["q_rope"], lat, r["kv_b"], r["dn"], r["dv"],
                                  offset=r["offset"], softmax_scale_mult=1.1)
    assert np.abs(wrong_scale - exp).max() > 1e-3
    no_rope_lat = lat.copy()
    no_rope_lat[..., -2:] = 0
    wrong_rope, _ = mla.absorbed(r["q_nope"], r["q_rope"], no_rope_lat, r["kv_b"], r["dn"],
                                 r["dv"], offset=r["offset"])
    assert np.abs(wrong_rope - exp).max() > 1e-3
    wrong_offset, _ = mla.absorbed(r["q_nope"], r["q_rope"], lat, r["kv_b"], r["dn"], r["dv"],
                                   offset=r["offset"] - 1)
    assert np.abs(wrong_offset - exp).max() > 1e-3


def test_decode_step_identity_at_config5_geometry_small_context():
    # L = 1 (decode), DeepSeek-V3 geometry dn=dv=128, dr=64, latent 512, a few heads.
    rng = np.random.default_rng(8)
    B, H, S, dn, dr, dv, C = 2, 4, 70, 128, 64, 128, 512
    q_nope = rng.standard_normal((B, H, 1, dn)).astype(np.float32)
    q_rope = rng.standard_normal((B, H, 1, dr)).astype(np.float32)
    c_all = rng.standard_normal((B, S, C)).astype(np.float32)
    k_rope = rng.standard_normal((B, S, dr)).astype(np.float32)
    kv_b = (rng.standard_normal((H * (dn + dv), C)) * 0.02).astype(np.float32)
    lat = np.concatenate([c_all, k_rope], axis=-1)
    exp = mla.expanded(q_nope, q_rope, c_all, k_rope, kv_b, dn, dv, offset=S - 1)
    got, _ = mla.absorbed(q_nope, q_rope, lat, kv_b, dn, dv, offset=S - 1)
    np.testing.assert_allclose(got, exp, atol=2e-5, rtol=2e-5)
    got_bf, _ = mla.absorbed(q_nope, q_rope, obf.round_bf16(lat), kv_b, dn, dv,
                             offset=S - 1, bf16=True)
    np.testing.assert_allclose(got_bf, exp, atol=2e-2, rtol=1e-2)


def test_bf16_rounding_is_round_to_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, np.inf, -np.inf], np.float32)
    r = obf.round_bf16(x)
    np.testing.assert_array_equal(r, np.array([1.0, 1.0, 1.0 + 2 ** -6, -2.5, np.inf, -np.inf],
                                              np.float32))
    assert np.isnan(obf.round_bf16(np.array([np.nan], np.float32)))[0]


def test_torch_cpu_contraction_matches_numpy_restatement():
    """The torch-CPU dense contraction (the timed CPU baseline) agrees with the
    pinned numpy restatement in bf16 mode up to one bf16 ulp of rounding-order
    differences in the fp32 sums."""
    import torch

    from oracle.bf16 import round_bf16

    rng = np.random.default_rng(3)
    B, H, S, C, dr = 2, 4, 70, 32, 8
    q_lat = round_bf16(rng.standard_normal((B, H, C + dr)).astype(np.float32))
    lat = round_bf16(rng.standard_normal((B, S, C + dr)).astype(np.float32))
    scale = (16 + dr) ** -0.5
    ref = mla.absorbed_weighted_c(q_lat[:, :, None], lat, dr, scale, bf16=True)[:, :, 0]
    got = mla.absorbed_weighted_c_torch(torch.from_numpy(q_lat).to(torch.bfloat16),
                                         torch.from_numpy(lat).to(torch.bfloat16), dr, scale)
    np.testing.assert_allclose(got.numpy(), ref, rtol=2 ** -7, atol=1e-3)
