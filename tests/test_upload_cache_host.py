"""The upload cache's budget and eviction order (host logic; the upload is
replaced by a stand-in, so no device is used): entries count rows * cols +
blocks * 8 bytes from insertion (crates/inference/kernels/src/gpu.rs:171-173),
the least recently used leave first, before the upload that needs the room
(gpu.rs:186-192), and an evicted matrix is not freed while a caller holds it."""
import numpy as np
import pytest

from iris_amd import tensor


class FakeMatrix:
    uploaded = []
    freed = []

    def __init__(self, key, rows, cols):
        self.key, self.rows, self.cols = key, rows, cols

    def __del__(self):
        FakeMatrix.freed.append(self.key)


@pytest.fixture
def fake_uploads(monkeypatch):
    FakeMatrix.uploaded, FakeMatrix.freed = [], []

    def from_bytes(raw, rows, cols):
        m = FakeMatrix(int(raw[0]), rows, cols)
        FakeMatrix.uploaded.append((m.key, len(cache_ref[0]) if cache_ref else 0))
        return m

    cache_ref = []
    monkeypatch.setattr(tensor.Q8Matrix, "from_bytes", staticmethod(from_bytes))
    return cache_ref


def test_budget_and_lru_order(fake_uploads):
    size = tensor.UploadCache.counted_bytes(16, 64)  # 16*64 + 16*2*8
    assert size == 1280
    cache = tensor.UploadCache(budget=3 * size)
    fake_uploads.append(cache)
    raw = [np.array([k], dtype=np.uint8) for k in range(6)]
    for k in range(3):
        cache.get(k, raw[k], 16, 64)
    assert cache.held == 3 * size and len(cache) == 3
    cache.get(0, raw[0], 16, 64)  # a hit: 0 becomes the most recent
    assert cache.uploads == 3
    cache.get(3, raw[3], 16, 64)  # evicts 1, the least recently used
    assert 1 not in cache and 0 in cache and 3 in cache
    assert cache.held == 3 * size
    # the eviction happened before the upload: the cache held 2 entries then
    assert FakeMatrix.uploaded[-1] == (3, 2)


def test_a_held_matrix_survives_eviction(fake_uploads):
    size = tensor.UploadCache.counted_bytes(16, 64)
    cache = tensor.UploadCache(budget=size)
    fake_uploads.append(cache)
    held = cache.get(7, np.array([7], dtype=np.uint8), 16, 64)
    cache.get(8, np.array([8], dtype=np.uint8), 16, 64)  # evicts 7 from the cache
    assert 7 not in cache and 7 not in FakeMatrix.freed
    del held
    assert 7 in FakeMatrix.freed


def test_an_entry_larger_than_the_budget_is_still_uploaded(fake_uploads):
    cache = tensor.UploadCache(budget=100)
    fake_uploads.append(cache)
    cache.get(1, np.array([1], dtype=np.uint8), 16, 64)
    cache.get(2, np.array([2], dtype=np.uint8), 16, 64)
    assert len(cache) == 1 and 2 in cache
