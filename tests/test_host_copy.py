"""The library's multi-threaded staging memcpy (cascade_host_copy and the
caller-owned cascade_copy_pool_*), on the CPU: it replaces the pageable ->
pinned tensor copy of the pinned-staging store (reference
layer_streaming/weight_store.py:258-268) and must equal that copy byte for
byte for any size and alignment."""

import os
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


@pytest.mark.parametrize("nbytes", [1, (2 << 20) + 17, (9 << 20) + 5])
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_copy_pool_equals_tensor_copy(nbytes, threads):
    gen = torch.Generator().manual_seed(nbytes * threads)
    src = torch.randint(0, 256, (nbytes + 7,), dtype=torch.uint8, generator=gen)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8)
    with _hip.CopyPool(threads) as pool:
        assert pool.threads == threads and pool.bound_cpus == 0
        for _ in range(2):  # the helpers serve one copy after another
            dst.zero_()
            pool.copy(dst[5:5 + nbytes], src[7:7 + nbytes])
            assert torch.equal(dst[5:5 + nbytes], src[7:7 + nbytes])
            assert int(dst[:5].sum()) == 0 and int(dst[5 + nbytes:].sum()) == 0


def _node_cpus(node):
    with open("/sys/devices/system/node/node{}/cpulist".format(node)) as f:
        cpus = set()
        for part in f.read().strip().split(","):
            lo, _, hi = part.partition("-")
            cpus.update(range(int(lo), int(hi or lo) + 1))
    return cpus & os.sched_getaffinity(0)


@pytest.mark.skipif(not os.path.exists("/sys/devices/system/node/node0/cpulist"),
                    reason="no NUMA topology in sysfs")
def test_copy_pool_binds_helpers_to_a_node():
    src = torch.arange(5 << 20, dtype=torch.int32)
    dst = torch.empty_like(src)
    with _hip.CopyPool(4, numa_node=0) as pool:
        assert pool.bound_cpus == len(_node_cpus(0))
        pool.copy(dst, src)
    assert torch.equal(dst, src)


@pytest.mark.skipif(not os.path.exists("/sys/devices/system/node/node0/cpulist"),
                    reason="no NUMA topology in sysfs")
def test_copy_pools_created_concurrently_bind_the_same_cpus():
    # the node's CPU list is parsed without shared parser state, so pools
    # made from several threads at once all see the whole list
    expected = len(_node_cpus(0))
    counts, errors = [], []
    start = threading.Barrier(8)

    def make():
        try:
            start.wait()
            for _ in range(20):
                with _hip.CopyPool(2, numa_node=0) as pool:
                    counts.append(pool.bound_cpus)
        except Exception as error:  # reported below
            errors.append(error)

    threads = [threading.Thread(target=make) for _ in range(8)]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join()
    assert not errors
    assert counts == [expected] * 160


def test_copy_pool_rejects_bad_arguments():
    with pytest.raises(_hip.HipCallError):  # no such NUMA node
        _hip.CopyPool(2, numa_node=4095)
    with pytest.raises(_hip.HipCallError):
        _hip.CopyPool(2, numa_node=-2)
    with pytest.raises(_hip.HipCallError):  # thread count out of range
        _hip.CopyPool(65)
    buf = torch.zeros(1024, dtype=torch.uint8)
    pool = _hip.CopyPool(2)
    with pytest.raises(_hip.HipCallError):  # overlapping ranges
        _hip.call("cascade_copy_pool_copy", pool.handle, buf.data_ptr(),
                  buf.data_ptr() + 16, 512)
    pool.close()
    pool.close()  # idempotent
    with pytest.raises(RuntimeError):
        pool.copy(buf[:10], buf[100:110])
    with pytest.raises(_hip.HipCallError):
        _hip.call("cascade_copy_pool_copy", 0, buf.data_ptr(),
                  buf.data_ptr() + 512, 256)


def test_copy_pool_is_destroyed_when_collected():
    import gc
    import weakref

    pool = _hip.CopyPool(3)
    finalizer = pool._finalizer
    ref = weakref.ref(pool)
    del pool
    gc.collect()
    assert ref() is None and not finalizer.alive  # native pool destroyed


@pytest.mark.parametrize("pooled", [False, True])
def test_host_copy_concurrent_callers(pooled):
    # the staging store calls from two worker threads at once
    srcs = [torch.full((5 << 20,), i, dtype=torch.int16) for i in range(6)]
    dsts = [torch.empty_like(s) for s in srcs]
    errors = []
    pool = _hip.CopyPool(4) if pooled else None

    def run(i):
        try:
            for _ in range(3):
                if pool is None:
                    _hip.host_copy(dsts[i], srcs[i], 4)
                else:
                    pool.copy(dsts[i], srcs[i])
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(6)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    if pool is not None:
        pool.close()
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


def test_pool_finalized_during_a_copy_leaves_that_copy_alone():
    # what interpreter exit does to a daemon staging thread's pool: the
    # finalizer runs while a copy is in progress; the copy completes, the
    # native pool is not destroyed under it, and later copies are refused
    src = torch.arange(96 << 20, dtype=torch.int32)  # 384 MiB, ~0.1 s on one thread
    dst = torch.zeros_like(src)
    pool = _hip.CopyPool(1)
    started, outcome = threading.Event(), []

    def copy():
        started.set()
        try:
            pool.copy(dst, src)
            outcome.append("done")
        except Exception as error:  # reported below
            outcome.append(error)

    thread = threading.Thread(target=copy)
    thread.start()
    started.wait()
    while pool._state.busy == 0 and thread.is_alive():
        pass  # until the copy is inside the native call (or already over)
    pool._finalizer()
    thread.join()
    assert outcome == ["done"]
    assert torch.equal(dst, src)
    assert pool.handle == 0
    with pytest.raises(RuntimeError, match="closed"):
        pool.copy(dst[:8], src[:8])
