"""KV-cache persistence through libpqa.so on the GPU: pqa_kvc_save /
pqa_kvc_load against the .kvc oracle (restating picolm/model.c:870-983), the
file the reference's kvcache_save wrote (tests/golden/kvc_ref_*.npz) and,
where it was built, the reference's compiled kvcache_save / kvcache_load.
Bit-exact throughout: file bytes, return values, and every cache byte after a
load (rows the file does not cover keep what they held)."""
import os

import numpy as np
import pytest

import oracle as O
from gpu_util import assert_bits_equal
from kvc_cases import load_cases, random_caches

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402
from picolm_qwen_amd._lib import PQA_ERR_IO, PQA_ERR_RANGE, PQAError  # noqa: E402

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "kvc_ref_l2_s8_kv128_pos5.npz")


def _ctx(n_layers, smax, nkv, hd):
    return PicoAttention(n_layers, smax, 2 * nkv, nkv, hd)


def _upload(att, k, v):
    for layer in range(k.shape[0]):
        att.kv_upload(layer, 0, k[layer], v[layer])


def _download(att):
    ks, vs = zip(*(att.kv_download(layer, 0, att.max_seq_len) for layer in range(att.n_layers)))
    return np.stack(ks), np.stack(vs)


def test_save_reproduces_reference_golden_file(tmp_path):
    g = np.load(GOLDEN)
    k, v, n_pos = g["key_cache"], g["val_cache"], int(g["n_pos"])
    att = _ctx(k.shape[0], k.shape[1], int(g["n_kv_heads"]), int(g["head_dim"]))
    _upload(att, k, v)
    path = tmp_path / "ours.kvc"
    att.kvc_save(str(path), n_pos)
    assert path.read_bytes() == g["kvc"].tobytes()
    att.close()


def test_load_of_reference_golden_file(tmp_path):
    g = np.load(GOLDEN)
    k, v, n_pos = g["key_cache"], g["val_cache"], int(g["n_pos"])
    att = _ctx(k.shape[0], k.shape[1], int(g["n_kv_heads"]), int(g["head_dim"]))
    path = tmp_path / "ref.kvc"
    path.write_bytes(g["kvc"].tobytes())
    assert att.kvc_load(str(path)) == n_pos
    gk, gv = _download(att)
    assert_bits_equal(gk[:, :n_pos], k[:, :n_pos], "K rows")
    assert_bits_equal(gv[:, :n_pos], v[:, :n_pos], "V rows")
    assert not gk[:, n_pos:].any() and not gv[:, n_pos:].any()
    att.close()


@pytest.mark.parametrize("n_pos", [1, 7, 10])
def test_save_matches_oracle_and_reference(tmp_path, n_pos):
    k, v = random_caches(np.random.default_rng(300 + n_pos), 3, 10, 128)
    att = _ctx(3, 10, 2, 64)
    _upload(att, k, v)
    path = tmp_path / "ours.kvc"
    att.kvc_save(str(path), n_pos)
    data = path.read_bytes()
    assert data == O.kvc_file_bytes(k, v, n_pos)
    if O.RefKvc.available():
        ref = tmp_path / "ref.kvc"
        assert O.RefKvc.save(k, v, 2, 64, ref, n_pos) == 0
        assert ref.read_bytes() == data
    att.close()


def test_save_rejects_bad_n_pos_without_creating_a_file(tmp_path):
    att = _ctx(2, 10, 2, 64)
    for n in (0, -3, 11):
        path = tmp_path / f"bad{n}.kvc"
        with pytest.raises(PQAError) as e:
            att.kvc_save(str(path), n)
        assert e.value.code == PQA_ERR_RANGE and not path.exists()
    with pytest.raises(PQAError) as e:
        att.kvc_save(str(tmp_path / "no_such_dir" / "x.kvc"), 3)
    assert e.value.code == PQA_ERR_IO
    att.close()


def test_load_matches_oracle_on_every_branch(tmp_path):
    rng = np.random.default_rng(91)
    k, v = random_caches(rng, 3, 10, 128)
    junk_k, junk_v = random_caches(rng, 3, 10, 128)
    att = _ctx(3, 10, 2, 64)
    for name, data in load_cases(k, v, 7):
        print(f"kvc load case {name}", flush=True)
        path = tmp_path / f"{name}.kvc"
        path.write_bytes(data)
        _upload(att, junk_k, junk_v)
        wk, wv = junk_k.copy(), junk_v.copy()
        want = O.kvc_load_bytes(data, wk, wv)
        got = att.kvc_load(str(path))
        assert got == want, (name, got, want, att.last_error())
        gk, gv = _download(att)
        assert_bits_equal(gk, wk, f"K cache after {name}")
        assert_bits_equal(gv, wv, f"V cache after {name}")
    assert att.kvc_load(str(tmp_path / "absent.kvc")) == 0
    assert "absent.kvc" in att.last_error()
    att.close()


def test_chunked_streaming_round_trip(tmp_path):
    # 6 runs of 3000 rows x 2 KiB = 36.9 MB: the 16 MiB staging chunks end
    # inside runs, and the cut file ends inside the second buffer's chunk.
    n_layers, smax, nkv, hd, n_pos = 3, 3072, 8, 128, 3000
    rng = np.random.default_rng(17)
    k, v = random_caches(rng, n_layers, smax, nkv * hd)
    att = _ctx(n_layers, smax, nkv, hd)
    _upload(att, k, v)
    path = tmp_path / "big.kvc"
    att.kvc_save(str(path), n_pos)
    data = path.read_bytes()
    want = O.kvc_file_bytes(k, v, n_pos)
    assert len(data) == len(want) and data == want
    del want

    junk_k, junk_v = random_caches(rng, n_layers, smax, nkv * hd)
    _upload(att, junk_k, junk_v)
    assert att.kvc_load(str(path)) == n_pos
    gk, gv = _download(att)
    assert_bits_equal(gk[:, :n_pos], k[:, :n_pos], "K rows")
    assert_bits_equal(gv[:, :n_pos], v[:, :n_pos], "V rows")
    assert_bits_equal(gk[:, n_pos:], junk_k[:, n_pos:], "K rows past n_pos")

    cut = tmp_path / "cut.kvc"
    cut.write_bytes(data[:16 + 20_000_001])
    _upload(att, junk_k, junk_v)
    wk, wv = junk_k.copy(), junk_v.copy()
    assert O.kvc_load_bytes(data[:16 + 20_000_001], wk, wv) == 0
    assert att.kvc_load(str(cut)) == 0
    gk, gv = _download(att)
    assert_bits_equal(gk, wk, "K cache after a cut file")
    assert_bits_equal(gv, wv, "V cache after a cut file")
    att.close()


def test_save_sees_rows_appended_by_queued_decode(tmp_path):
    # Decode calls are queued on the context stream without a sync; the save
    # must order after them and write the rows they appended.
    nh, nkv, hd, smax, hist = 4, 2, 64, 64, 10
    att = PicoAttention(1, smax, nh, nkv, hd, 0, 1e6)
    att.synth_kv(0, 0, hist, 55, 0.0)
    dev = torch.device("cuda:0")
    for i, pos in enumerate(range(hist, hist + 3)):
        q, k, v = O.step_inputs(55, 0, i, nh, nkv, hd)
        att.forward(0, pos, torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
    path = tmp_path / "after_decode.kvc"
    att.kvc_save(str(path), hist + 3)
    gk, gv = att.kv_download(0, 0, smax)
    assert path.read_bytes() == O.kvc_file_bytes(gk[None], gv[None], hist + 3)
    assert gk[hist:hist + 3].any()
    att.close()


def test_loaded_cache_decodes_like_the_original(tmp_path):
    # The reference's use: load a prompt's cache and continue at n_pos. The
    # decode output after a load equals the one over the cache it was saved
    # from, bit for bit (same kernels, same bytes).
    nh, nkv, hd, smax, n_pos = 16, 8, 128, 512, 300
    a = PicoAttention(2, smax, nh, nkv, hd, 0, 1e6)
    b = PicoAttention(2, smax, nh, nkv, hd, 0, 1e6)
    for layer in range(2):
        a.synth_kv(layer, 0, n_pos, 900 + layer, 0.0)
    path = tmp_path / "prompt.kvc"
    a.kvc_save(str(path), n_pos)
    assert b.kvc_load(str(path)) == n_pos
    dev = torch.device("cuda:0")
    for layer in range(2):
        q, k, v = (torch.from_numpy(x).to(dev) for x in O.step_inputs(901, layer, 0, nh, nkv, hd))
        oa = a.forward(layer, n_pos, q, k, v).cpu().numpy()
        ob = b.forward(layer, n_pos, q, k, v).cpu().numpy()
        assert_bits_equal(oa.view(np.uint32), ob.view(np.uint32), f"layer {layer} output")
    a.close()
    b.close()
