"""Host codec and oracle against known answers of the reference's own host
code (tests/golden/reference_host.npz, written by tests/golden/make_golden.py
from oracle/_ref) and against closed forms of the mathematics."""
import numpy as np
import pytest
from scipy.linalg import hadamard

from oracle import oracle as orc


def test_flip_bytes_match_reference(chimera_mod, golden):
    for seed in (42, 7, 123456789):
        assert np.array_equal(chimera_mod._rotator_flips(seed, 128), golden[f"flips_seed{seed}"])


@pytest.mark.parametrize("dim", [64, 96, 100, 128])
def test_rotation_bit_exact(chimera_mod, golden, dim):
    flips = golden["flips_seed42"]
    x, y = golden[f"rot_in_d{dim}"], golden[f"rot_out_d{dim}"]
    assert np.array_equal(chimera_mod._rotate(x, flips), y)
    assert np.array_equal(orc.rotate(x, flips), y)


def test_rotation_closed_form(golden):
    # D=128: x <- (1/sqrt(128)) H D_r x for r = 0..3 with the Sylvester Hadamard
    # matrix and the sign flips of round r (bit j%8 of byte j/8 of its 16 bytes).
    flips = golden["flips_seed42"]
    H = hadamard(128).astype(np.float64)
    x = golden["rot_in_d128"].astype(np.float64)
    for r in range(4):
        fb = flips[16 * r:16 * r + 16]
        sign = np.array([-1.0 if (fb[j >> 3] >> (j & 7)) & 1 else 1.0 for j in range(128)])
        x = (x * sign) @ H.T / np.sqrt(128.0)
    np.testing.assert_allclose(golden["rot_out_d128"], x, rtol=0, atol=2e-6)
    # orthogonal: norms preserved
    np.testing.assert_allclose(np.linalg.norm(golden["rot_out_d128"], axis=1),
                               np.linalg.norm(golden["rot_in_d128"], axis=1), rtol=1e-5)


def test_one_bit_encoder(chimera_mod, golden):
    codes, f = chimera_mod._encode_one_bit(golden["enc_in"])
    assert np.array_equal(codes, golden["onebit_codes"])
    # factor differs from Eigen's vectorised dot only in rounding
    np.testing.assert_allclose(f, golden["onebit_factors"], rtol=2e-6)


@pytest.mark.parametrize("b", range(1, 8))
def test_full_code_encoder(chimera_mod, golden, b):
    enc = golden["enc_in"]
    assert np.array_equal(chimera_mod._quantize_ex(enc, b), golden[f"exq_b{b}"])
    packed, f = chimera_mod._encode_full(enc, b)
    assert np.array_equal(packed, golden[f"full_b{b}"])
    np.testing.assert_allclose(f, golden[f"full_f_b{b}"], rtol=2e-6)


@pytest.mark.parametrize("w", range(1, 9))
def test_pack_unpack(chimera_mod, golden, w):
    raw, pk = golden[f"pack_raw_w{w}"], golden[f"pack_w{w}"]
    assert np.array_equal(chimera_mod._pack(raw, w), pk)
    assert np.array_equal(chimera_mod._unpack(pk, w), raw)
    assert np.array_equal(orc.unpack(pk, w), raw)
    if w >= 2:
        assert np.array_equal(golden[f"unpack_w{w}"], raw.astype(np.float32))


@pytest.mark.parametrize("w", range(1, 9))
def test_pack_roundtrip_every_value(chimera_mod, w):
    # every value in every lane position
    vals = np.arange(1 << w, dtype=np.uint8)
    raw = np.stack([np.roll(np.resize(vals, 128), s) for s in range(max(1, 1 << w))]).astype(np.uint8)
    assert np.array_equal(chimera_mod._unpack(chimera_mod._pack(raw, w), w), raw)
    assert np.array_equal(orc.unpack(chimera_mod._pack(raw, w), w), raw)


@pytest.mark.parametrize("b", range(1, 8))
def test_full_bit_score_matches_reference_loop(golden, b):
    """The oracle's SF equals compute_full_bit_scores bit for bit."""
    ptrs = golden["fb_doc_ptrs"]
    n = int(ptrs[-1])
    index = orc.Index({
        "num_embeddings": n, "dimension": 128, "num_clusters": 1, "ex_bits": b,
        "doc_lens": np.diff(ptrs).astype(np.int32), "doc_ptrs": ptrs,
        "cluster_pos": np.array([0, n], np.uint64), "clustered_codes": np.zeros(n * 16, np.uint8),
        "clustered_factors": np.zeros(n, np.float32), "clustered_doc_ids": np.zeros(n, np.int32),
        "token_to_cluster_pos": np.arange(n, dtype=np.uint32),
        "full_bit_codes": golden[f"fb_codes_b{b}"].reshape(-1), "full_bit_factors": golden[f"fb_factors_b{b}"],
        "rotated_centroids": np.zeros(128, np.float32), "flips": golden["flips_seed42"],
    })
    docs = np.arange(ptrs.size - 1, dtype=np.int32)[None, :]
    got = orc.full_bit_scores(index, golden["fb_query_rot"][None], golden[f"fb_cbex_b{b}"][None], docs)
    assert np.array_equal(got[0], golden[f"fb_scores_b{b}"])


def test_query_state_and_lut_closed_form(golden):
    rot = golden["enc_in"]
    cb1, cbex = orc.query_state(rot, 4)
    s = rot.astype(np.float64).sum(1)
    np.testing.assert_allclose(cb1, s / 2, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cbex, s * 31 / 2, rtol=1e-5, atol=1e-5)
    lut = orc.lut(rot)
    # lut[i, c, e] = sum of rot[i, 4c + b] over the set bits b of e
    bits = ((np.arange(16)[:, None] >> np.arange(4)[None, :]) & 1).astype(np.float64)  # [16, 4]
    expect = np.einsum("icb,eb->ice", rot.reshape(32, 32, 4).astype(np.float64), bits)
    np.testing.assert_allclose(lut, expect, atol=1e-6)
    # the sequential-sum identity: sum over chunks of lut[nibble] = <bits, rot>
    code = golden["onebit_codes"]
    for i in range(4):
        b = np.array([(int(code[i, j // 64]) >> (j % 64)) & 1 for j in range(128)], np.float64)
        ip = sum(lut[i, c, sum(int(b[4 * c + k]) << k for k in range(4))] for c in range(32))
        assert abs(ip - float(b @ rot[i])) < 1e-5
