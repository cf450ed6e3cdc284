"""The library's multi-threaded staging memcpy (cascade_host_copy), on the
CPU: it replaces the pageable -> pinned tensor copy of the pinned-staging
store (reference layer_streaming/weight_store.py:258-268) and must equal
that copy byte for byte for any size and alignment."""

import threading

import pytest
import torch

from layer_streaming import _hip


@pytest.mark.parametrize("nbytes", [1, 31, 32, 129, 4096, (2 << 20) - 1,
                                    (2 << 20) + 17, (9 << 20) + 5])
@pytest.mark.parametrize("src_off,dst_off", [(0, 0), (1, 3), (7, 0), (0, 13)])
def test_host_copy_equals_tensor_copy(nbytes, src_off, dst_off):
    gen = torch.Generator().manual_seed(nbytes + src_off)
    src = torch.randint(0, 256, (nbytes + 64,), dtype=torch.uint8, generator=gen)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8)
    _hip.host_copy(dst[dst_off:dst_off + nbytes], src[src_off:src_off + nbytes], 8)
    assert torch.equal(dst[dst_off:dst_off + nbytes], src[src_off:src_off + nbytes])
    # nothing outside the destination range was written
    assert int(dst[:dst_off].sum()) == 0
    assert int(dst[dst_off + nbytes:].sum()) == 0


@pytest.mark.parametrize("threads", [1, 2, 5, 16])
def test_host_copy_thread_counts(threads):
    src = torch.arange(3 << 20, dtype=torch.int32)
    dst = torch.empty_like(src)
    _hip.host_copy(dst, src, threads)
    assert torch.equal(dst, src)


def test_host_copy_concurrent_callers():
    # the staging store calls from two worker threads at once
    srcs = [torch.full((5 << 20,), i, dtype=torch.int16) for i in range(6)]
    dsts = [torch.empty_like(s) for s in srcs]
    errors = []

    def run(i):
        try:
            for _ in range(3):
                _hip.host_copy(dsts[i], srcs[i], 4)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(6)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    for s, d in zip(srcs, dsts):
        assert torch.equal(s, d)


def test_host_copy_rejects_bad_arguments():
    buf = torch.zeros(1024, dtype=torch.uint8)
    with pytest.raises(_hip.HipCallError):  # overlapping ranges
        _hip.call("cascade_host_copy", buf.data_ptr(), buf.data_ptr() + 16, 512, 2)
    with pytest.raises(_hip.HipCallError):  # thread count out of range
        _hip.call("cascade_host_copy", buf.data_ptr(), buf.data_ptr() + 512, 256, 0)
    with pytest.raises(ValueError):  # size mismatch
        _hip.host_copy(buf[:10], buf[100:120])
    with pytest.raises(ValueError):  # not contiguous
        _hip.host_copy(buf[:10], buf[100:120:2])
