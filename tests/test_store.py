"""The host expert store (wisp/store.py): the `.u8` row file (reference store.py:62-67,
96-110: rows back to back, no header) round-trips byte for byte, reads files laid out as the
reference writes them, refuses a file of the wrong size; on the GPU, `fill` writes the
oracle's quantized bytes into the right rows."""

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from wisp.store import ExpertStore


def _random_store(L, E, n, bits, group, seed):
    st = ExpertStore(L, E, n, bits, group, pin=False)
    g = torch.Generator().manual_seed(seed)
    st.host.copy_(torch.randint(0, 256, st.host.shape, generator=g, dtype=torch.uint8))
    return st


def test_save_load_round_trip(tmp_path):
    st = _random_store(3, 5, 256 * 128, 4, 128, seed=1)
    assert st.host.shape == (15, O.expert_nbytes(256 * 128, 4, 128)) and not st.pinned
    path = str(tmp_path / "s.u8")
    st.save(path)
    assert os.path.getsize(path) == st.host.numel() and not os.path.exists(path + ".tmp")
    # the file is the rows back to back (the reference's format): compare with numpy's raw dump
    assert open(path, "rb").read() == st.host.numpy().tobytes()
    back = ExpertStore(3, 5, 256 * 128, 4, 128, pin=False)
    back.load(path)
    assert torch.equal(back.host, st.host)


def test_loads_a_file_written_row_block_by_row_block(tmp_path):
    # the reference writes 256-row blocks one after another (store.py:96-102): same bytes
    st = _random_store(2, 300, 64 * 32, 3, 32, seed=2)
    path = str(tmp_path / "ref.u8")
    a = st.host.numpy()
    with open(path, "wb") as f:
        for i in range(0, a.shape[0], 256):
            f.write(memoryview(a[i : i + 256]))
    back = ExpertStore(2, 300, 64 * 32, 3, 32, pin=False)
    back._load(path)
    assert torch.equal(back.host, st.host)
    other = str(tmp_path / "mine.u8")
    back._save(other)
    assert open(other, "rb").read() == open(path, "rb").read()


def test_load_refuses_a_file_of_another_shape(tmp_path):
    st = _random_store(1, 4, 256 * 128, 4, 128, seed=3)
    path = str(tmp_path / "s.u8")
    st.save(path)
    wrong = ExpertStore(1, 5, 256 * 128, 4, 128, pin=False)
    with pytest.raises(ValueError, match="bytes"):
        wrong.load(path)


def test_store_rows_and_cache_name():
    st = ExpertStore(4, 128, 2048 * 768, 4, 128, pin=False)
    assert st.nbytes == 2506752 and st.rows == 512 and st.key(3, 7) == 3 * 128 + 7
    assert abs(st.total_gib - 512 * 2506752 / 2**30) < 1e-9
    assert ExpertStore.cache_file("/c", 4, 128, 48, 128, 2048 * 768) == "/c/store_b4_g128_48x128x1572864.u8"


def test_fill_rejects_a_key_outside_the_store():
    st = ExpertStore(1, 2, 64 * 32, 4, 32, pin=False)
    with pytest.raises(IndexError):
        st.fill([(2, torch.zeros(3, 64 * 32))], device="cpu")


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 3, 2, 8])
def test_fill_writes_the_oracle_bytes(bits):
    H, I, G, L, E = 256, 128, 128, 2, 5
    n = H * I
    rng = np.random.default_rng(bits)
    w = {(l, e): (rng.standard_normal(3 * n) * 0.05).astype(np.float32) for l in range(L) for e in range(E)}
    st = ExpertStore(L, E, n, bits, G, pin=True)
    st.host.fill_(0xAB)
    order = [(1, 4), (0, 0), (1, 1), (0, 3), (1, 0), (0, 1), (0, 2)]  # not row order; ring of 4 wraps
    got = st.fill(((st.key(l, e), torch.from_numpy(w[l, e]).view(3, n)) for l, e in order), "cuda", ring=4)
    assert got == len(order)
    for l, e in order:
        assert np.array_equal(st.host[st.key(l, e)].numpy(), O.quantize(w[l, e], bits, G)), (l, e)
    untouched = [st.key(l, e) for l in range(L) for e in range(E) if (l, e) not in order]
    assert all(bool((st.host[k] == 0xAB).all()) for k in untouched)
    st.put(1, 2, torch.from_numpy(w[1, 2]).view(3, n).cuda())
    assert np.array_equal(st.host[st.key(1, 2)].numpy(), O.quantize(w[1, 2], bits, G))
