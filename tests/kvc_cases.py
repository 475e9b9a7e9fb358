"""Input files for the .kvc load tests: every branch of kvcache_load
(picolm/model.c:923-983), built from valid files by editing the header or
cutting the body. Shared by the oracle tests and the GPU tests."""
import numpy as np

import oracle as O


def random_caches(rng, n_layers, max_seq_len, kv_dim):
    shape = (n_layers, max_seq_len, kv_dim)
    return (rng.integers(0, 1 << 16, shape, dtype=np.uint16), rng.integers(0, 1 << 16, shape, dtype=np.uint16))


def with_header(data, index, value):
    h = np.frombuffer(data[:16], dtype="<u4").copy()
    h[index] = value
    return h.tobytes() + data[16:]


def load_cases(k, v, n_pos):
    """(name, file bytes) pairs; k/v are [n_layers][max_seq_len][kv_dim] uint16."""
    n_layers, max_seq_len, kv_dim = k.shape
    good = O.kvc_file_bytes(k, v, n_pos)
    full = O.kvc_file_bytes(k, v, max_seq_len)
    run = n_pos * kv_dim * 2
    return [
        ("valid", good),
        ("valid_full", full),
        ("valid_one_row", O.kvc_file_bytes(k, v, 1)),
        ("trailing_bytes", good + b"\x5a" * 7),
        ("bad_magic", with_header(good, 0, O.KVC_MAGIC ^ 0x100)),
        ("layers_mismatch", with_header(good, 2, n_layers + 1)),
        ("kv_dim_mismatch", with_header(good, 3, kv_dim // 2)),
        ("n_pos_exceeds_max_seq_len", with_header(full + full[16:16 + 2 * n_layers * kv_dim * 2], 1,
                                                  max_seq_len + 1)),
        ("n_pos_zero", with_header(good, 1, 0)),
        ("n_pos_all_ones", with_header(good, 1, 0xFFFFFFFF)),
        ("n_pos_2_pow_31", with_header(good, 1, 0x80000000)),
        ("empty", b""),
        ("short_header", good[:10]),
        ("header_only", good[:16]),
        ("cut_mid_row_k", good[:16 + run // 3 + 5]),
        ("cut_at_run_boundary", good[:16 + run]),
        ("cut_in_v", good[:16 + n_layers * run + 3 * kv_dim * 2 + 1]),
        ("cut_last_byte", good[:-1]),
    ]
