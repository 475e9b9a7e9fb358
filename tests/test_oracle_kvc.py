"""The .kvc oracle (oracle.kvc_file_bytes / kvc_load_bytes, restating
picolm/model.c:870-983) pinned three ways: the format's closed form, a file
written by the reference's kvcache_save (tests/golden/kvc_ref_*.npz), and the
reference's compiled kvcache_save / kvcache_load on every branch of both."""
import os

import numpy as np
import pytest

import oracle as O
from kvc_cases import load_cases, random_caches

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "kvc_ref_l2_s8_kv128_pos5.npz")

needs_ref = pytest.mark.skipif(not O.RefKvc.available(), reason="oracle/_ref/libref_kvc.so not built")


def test_closed_form_layout():
    # Header = four little-endian uint32, "PCVK" on disk; then layer-major K
    # rows, then V rows; length 16 + 2 * n_layers * n_pos * kv_dim * 2.
    rng = np.random.default_rng(5)
    k, v = random_caches(rng, 3, 11, 64)
    data = O.kvc_file_bytes(k, v, 4)
    assert len(data) == 16 + 2 * 3 * 4 * 64 * 2
    assert data[:4] == b"PCVK"
    assert data[4:16] == bytes([4, 0, 0, 0, 3, 0, 0, 0, 64, 0, 0, 0])
    # row p of layer l of K starts at 16 + (l*n_pos + p)*row; of V after all of K
    row = 64 * 2
    for layer, p in [(0, 0), (1, 3), (2, 1)]:
        at = 16 + (layer * 4 + p) * row
        assert data[at:at + row] == k[layer, p].astype("<u2").tobytes()
        at = 16 + 3 * 4 * row + (layer * 4 + p) * row
        assert data[at:at + row] == v[layer, p].astype("<u2").tobytes()


def test_save_rejects_n_pos_outside_range():
    k, v = random_caches(np.random.default_rng(1), 2, 6, 64)
    for n in (0, -1, 7):
        assert O.kvc_file_bytes(k, v, n) is None


def test_round_trip_restores_rows_and_keeps_the_rest():
    rng = np.random.default_rng(8)
    k, v = random_caches(rng, 4, 9, 128)
    dk, dv = random_caches(rng, 4, 9, 128)
    before_k, before_v = dk.copy(), dv.copy()
    assert O.kvc_load_bytes(O.kvc_file_bytes(k, v, 6), dk, dv) == 6
    assert np.array_equal(dk[:, :6], k[:, :6]) and np.array_equal(dv[:, :6], v[:, :6])
    assert np.array_equal(dk[:, 6:], before_k[:, 6:]) and np.array_equal(dv[:, 6:], before_v[:, 6:])


def test_golden_file_from_reference_kvcache_save():
    g = np.load(GOLDEN)
    k, v, n_pos = g["key_cache"], g["val_cache"], int(g["n_pos"])
    assert O.kvc_file_bytes(k, v, n_pos) == g["kvc"].tobytes()
    dk, dv = np.zeros_like(k), np.zeros_like(v)
    assert O.kvc_load_bytes(g["kvc"].tobytes(), dk, dv) == n_pos
    assert np.array_equal(dk[:, :n_pos], k[:, :n_pos]) and not dk[:, n_pos:].any()
    assert np.array_equal(dv[:, :n_pos], v[:, :n_pos]) and not dv[:, n_pos:].any()


@needs_ref
@pytest.mark.parametrize("n_pos", [1, 3, 10, 0, -1, 11])
def test_save_matches_reference(tmp_path, n_pos):
    k, v = random_caches(np.random.default_rng(40 + n_pos), 3, 10, 128)
    path = tmp_path / "ref.kvc"
    rc = O.RefKvc.save(k, v, 2, 64, path, n_pos)
    ours = O.kvc_file_bytes(k, v, n_pos)
    if ours is None:
        assert rc == -1 and not path.exists()
    else:
        assert rc == 0 and path.read_bytes() == ours


@needs_ref
def test_load_matches_reference_on_every_branch(tmp_path):
    rng = np.random.default_rng(77)
    k, v = random_caches(rng, 3, 10, 128)
    junk_k, junk_v = random_caches(rng, 3, 10, 128)
    for name, data in load_cases(k, v, 7):
        path = tmp_path / f"{name}.kvc"
        path.write_bytes(data)
        rk, rv = junk_k.copy(), junk_v.copy()
        ok, ov = junk_k.copy(), junk_v.copy()
        r_ref = O.RefKvc.load_into(rk, rv, 2, 64, path)
        r_ours = O.kvc_load_bytes(data, ok, ov)
        assert r_ours == r_ref, name
        assert np.array_equal(ok, rk) and np.array_equal(ov, rv), name


@needs_ref
def test_load_of_missing_file_returns_zero(tmp_path):
    k, v = random_caches(np.random.default_rng(2), 2, 4, 128)
    assert O.RefKvc.load_into(k, v, 2, 64, tmp_path / "absent.kvc") == 0


def test_mistakes_are_caught():
    # A restatement with V written before K, or row-major over layers, must
    # differ from the reference file on the golden case.
    g = np.load(GOLDEN)
    k, v, n_pos = g["key_cache"], g["val_cache"], int(g["n_pos"])
    good = g["kvc"].tobytes()
    head = good[:16]
    v_first = head + v[:, :n_pos].tobytes() + k[:, :n_pos].tobytes()
    row_major = head + k[:, :n_pos].transpose(1, 0, 2).tobytes() + v[:, :n_pos].transpose(1, 0, 2).tobytes()
    assert v_first != good and row_major != good
