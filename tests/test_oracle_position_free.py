"""Pins oracle/position_free.py (a restatement of runtime/pic_attention.py)
with what the mathematics fixes, independently of the restatement:
  * the rotation equals multiplication by e^{i*angle} of the complex pairs
    (k[d] + i k[d + D/2]);
  * RoPE scores depend only on query position - key position;
  * keys past a query's position never contribute, and no visible key gives 0;
  * a block table that repeats page ids equals the gathered copy;
  * with every key visible it is plain softmax attention over rotated keys
    (fp64 brute force)."""
import numpy as np

from oracle import position_free as pf
from oracle import paged_attention as opa


def test_tables_are_the_textbook_angles():
    cos, sin = pf.rope_tables(40, 16, 10000.0)
    pos, i = 37, 5
    ang = pos / 10000.0 ** (i / 8)
    assert abs(cos[pos, i] - np.cos(ang)) < 1e-6 and abs(sin[pos, i] - np.sin(ang)) < 1e-6


def test_rotation_is_complex_multiplication():
    rng = np.random.default_rng(0)
    D = 64
    cos, sin = pf.rope_tables(300, D, 10000.0)
    k = rng.standard_normal((5, D)).astype(np.float32)
    pos = np.array([0, 1, 17, 128, 299])
    got = pf.rotate(k, pos, cos, sin, bf16=False)
    z = (k[:, :32] + 1j * k[:, 32:]) * (cos[pos] + 1j * sin[pos])
    np.testing.assert_allclose(got[:, :32], z.real, atol=1e-5)
    np.testing.assert_allclose(got[:, 32:], z.imag, atol=1e-5)
    assert np.array_equal(pf.rotate(k, np.zeros(5, int), cos, sin, bf16=False), k)


def test_scores_depend_only_on_relative_position():
    rng = np.random.default_rng(1)
    D = 64
    cos, sin = pf.rope_tables(2000, D, 10000.0)
    qraw = rng.standard_normal((1, D)).astype(np.float32)
    k = rng.standard_normal((8, D)).astype(np.float32)
    kpos = np.arange(8) * 3
    base = None
    for shift in (0, 500, 1500):
        q = pf.rotate(qraw, np.array([30 + shift]), cos, sin, bf16=False)
        kr = pf.rotate(k, kpos + shift, cos, sin, bf16=False)
        s = (q @ kr.T)[0]
        if base is None:
            base = s
        np.testing.assert_allclose(s, base, atol=2e-3)


def _case(rng, B=1, NQ=4, NKV=2, TQ=2, D=64, BLOCK=4, TK=23, P=12):
    q = rng.standard_normal((B, NQ, TQ, D)).astype(np.float32)
    kp = rng.standard_normal((P, NKV, BLOCK, D)).astype(np.float32)
    vp = rng.standard_normal((P, NKV, BLOCK, D)).astype(np.float32)
    table = rng.integers(0, P, size=(TK + BLOCK - 1) // BLOCK)
    return q, kp, vp, table


def test_causal_mask_and_empty_rows():
    rng = np.random.default_rng(2)
    q, kp, vp, _ = _case(rng)
    table = rng.permutation(12)[:6]  # distinct pages: poisoning one key touches no other
    cos, sin = pf.rope_tables(64, 64, 10000.0)
    kpos = np.arange(23)
    qpos = np.array([10, 22])
    out = pf.attention(q, kp, vp, table, kpos, qpos, cos, sin, 0.125)
    # poison the values of keys 11.. for query 0: its output must not move
    vp2 = vp.copy()
    for key in range(11, 23):
        vp2[table[key // 4], :, key % 4] = 1e6
    out2 = pf.attention(q, kp, vp2, table, kpos, qpos, cos, sin, 0.125)
    np.testing.assert_array_equal(out[:, :, 0], out2[:, :, 0])
    none = pf.attention(q, kp, vp, table, np.full(23, 50), np.array([10, 20]), cos, sin, 0.125)
    assert np.all(none == 0)


def test_repeated_page_ids_equal_the_gathered_copy():
    rng = np.random.default_rng(3)
    q, kp, vp, _ = _case(rng, P=3)
    table = np.array([2, 0, 2, 1, 0, 2])
    cos, sin = pf.rope_tables(64, 64, 10000.0)
    kpos = np.arange(23)
    qpos = np.array([22, 22])
    out = pf.attention(q, kp, vp, table, kpos, qpos, cos, sin, 0.1)
    kg = kp[table].copy()
    vg = vp[table].copy()
    out2 = pf.attention(q, kg, vg, np.arange(6), kpos, qpos, cos, sin, 0.1)
    np.testing.assert_array_equal(out, out2)


def test_all_visible_is_softmax_attention_over_rotated_keys():
    rng = np.random.default_rng(4)
    q, kp, vp, table = _case(rng, B=2, NQ=6, NKV=3, TQ=1, BLOCK=1, TK=30, P=40)
    cos, sin = pf.rope_tables(64, 64, 10000.0)
    kpos = rng.permutation(40)[:30]
    qpos = np.array([63])
    out = pf.attention(q, kp, vp, table, kpos, qpos, cos, sin, 0.125, bf16=False)
    for b in range(2):
        for kvh in range(3):
            krow = kp[table, kvh, 0]
            vrow = vp[table, kvh, 0]
            kr = pf.rotate(krow, kpos, cos, sin, bf16=False).astype(np.float64)
            qq = q[b, 2 * kvh:2 * kvh + 2, 0].astype(np.float64)
            ref = opa.sdpa_decode(qq, kr[None], vrow[None].astype(np.float64), 0.125)
            np.testing.assert_allclose(out[b, 2 * kvh:2 * kvh + 2, 0], ref, atol=1e-5)


def test_fp64_accumulation_matches_a_complex_rotation_brute_force():
    """store="f32", acc=float64 (the reference for fp32 pages) against an
    independent fp64 computation: keys rotated by complex multiplication,
    masked softmax by explicit loops."""
    rng = np.random.default_rng(5)
    q, kp, vp, table = _case(rng, B=1, NQ=4, NKV=2, TQ=3, D=64, BLOCK=4, TK=19, P=5)
    cos, sin = pf.rope_tables(32, 64, 10000.0)
    kpos = np.arange(19)
    qpos = np.array([5, 17, 18])
    out = pf.attention(q, kp, vp, table, kpos, qpos, cos, sin, 0.125, store="f32",
                       acc=np.float64)
    for h in range(4):
        kvh = h // 2
        for t in range(3):
            num = np.zeros(64)
            den = 0.0
            scores = []
            for key in range(19):
                if kpos[key] > qpos[t]:
                    continue
                krow = kp[table[key // 4], kvh, key % 4].astype(np.float64)
                z = (krow[:32] + 1j * krow[32:]) * np.exp(1j * np.arctan2(
                    sin[kpos[key]].astype(np.float64), cos[kpos[key]].astype(np.float64)))
                kr = np.concatenate([z.real, z.imag])
                scores.append((float(q[0, h, t].astype(np.float64) @ kr) * 0.125, key))
            m = max(s for s, _ in scores)
            for s, key in scores:
                w = np.exp(s - m)
                num += w * vp[table[key // 4], kvh, key % 4].astype(np.float64)
                den += w
            np.testing.assert_allclose(out[0, h, t], num / den, atol=2e-6)


def test_half_store_rounds_the_rotated_keys_to_fp16():
    rng = np.random.default_rng(6)
    cos, sin = pf.rope_tables(50, 64, 10000.0)
    k = rng.standard_normal((7, 64)).astype(np.float32)
    pos = np.arange(40, 47)
    full = pf.rotate(k, pos, cos, sin, store="f32")
    half = pf.rotate(k, pos, cos, sin, store="f16")
    assert np.array_equal(half, half.astype(np.float16).astype(np.float32))  # representable
    assert np.all(np.abs(half - full) <= np.abs(full) * 2.0 ** -11 + 2.0 ** -25)
    assert not np.array_equal(half, full)


def test_torch_cpu_restatement_matches_numpy():
    """The torch-CPU attention (the timed CPU baseline) agrees with the pinned
    numpy restatement, masked rows and repeated pages included."""
    import torch

    rng = np.random.default_rng(7)
    q, kp, vp, table = _case(rng, B=2, NQ=6, NKV=3, TQ=3, D=64, BLOCK=4, TK=23, P=6)
    cos, sin = pf.rope_tables(64, 64, 10000.0)
    kpos = np.arange(23)
    qpos = np.array([0, 10, 22])
    ref = pf.attention(q, kp, vp, table, kpos, qpos, cos, sin, 0.125, store="f32")
    got = pf.attention_torch(*(torch.from_numpy(np.ascontiguousarray(x)) for x in
                               (q, kp, vp, table, kpos, qpos, cos, sin)), 0.125)
    np.testing.assert_allclose(got.numpy(), ref, atol=2e-5)
    none = pf.attention_torch(*(torch.from_numpy(np.ascontiguousarray(x)) for x in
                                (q, kp, vp, table, np.full(23, 50), qpos, cos, sin)), 0.125)
    assert torch.all(none == 0)
