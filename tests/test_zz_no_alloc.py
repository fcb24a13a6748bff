"""chimera_search_device_noalloc (the search on the library's static device
workspace) against chimera_search_device through the C ABI: identical ids,
scores and counts on two calls in a row, the second with a smaller batch
(the static workspace keeps the first call's contents), in both scoring
modes; the first batch has 16 queries (512 probe rows), the second 3, after
a warm-up call that loads the kernels' code. The call allocates nothing:
the device's free memory and the context's own memory are the same before
and after it. A batch beyond the static
workspace is rejected with a capacity error that names the largest batch
that fits."""
import re

import numpy as np
import pytest

from chimera_amd import capi

pytestmark = pytest.mark.gpu


def run(ctx, fn, queries, k, bufs=None):
    nq = queries.shape[0]
    own = bufs is None
    if own:
        bufs = (ctx.to_device(queries), ctx.empty((nq, k), np.int64), ctx.empty((nq, k), np.float32),
                ctx.empty((nq,), np.int32))
    d_q, d_ids, d_sc, d_cnt = bufs
    try:
        fn(d_q, nq, k, d_ids, d_sc, d_cnt)
        ctx.synchronize()
        return d_ids.numpy(), d_sc.numpy(), d_cnt.numpy()
    finally:
        if own:
            for a in bufs:
                a.free()


@pytest.mark.parametrize("exact", [False, True], ids=["mfma", "exact"])
def test_noalloc_search_equals_search_device(small_index, small_workload, exact):
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=exact)
    print(f"no-alloc search: small index, exact={exact}, batches of 16 then 3 queries", flush=True)
    # one call first, so that loading the kernels' code is not counted below
    warm = np.ascontiguousarray(small_workload.queries[:2], np.float32)
    run(ctx, ctx.search_device_noalloc, warm, 10)
    for nq, k in ((16, 50), (3, 20)):
        q = np.ascontiguousarray(small_workload.queries[16 - nq:], np.float32)
        want = run(ctx, ctx.search_device, q, k)
        bufs = (ctx.to_device(q), ctx.empty((nq, k), np.int64), ctx.empty((nq, k), np.float32),
                ctx.empty((nq,), np.int32))
        try:
            free0, _ = ctx.device_memory_info()
            used0 = ctx.memory_usage()
            got = run(ctx, ctx.search_device_noalloc, q, k, bufs)
            free1, _ = ctx.device_memory_info()
            assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"
            assert ctx.memory_usage() == used0
        finally:
            for a in bufs:
                a.free()
        assert np.array_equal(got[2], want[2])
        assert np.array_equal(got[0], want[0])
        assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))
    ctx.close()


def test_noalloc_rejects_a_batch_beyond_the_static_workspace(small_index, small_workload):
    # nprobe 1024 of 1024 clusters: every query visits every token, so a few
    # queries' visit records exceed the static workspace
    ctx = capi.Context(small_index, 1024, 500, 100, 5, max_batch=16)
    q = np.ascontiguousarray(small_workload.queries, np.float32)
    with pytest.raises(capi.ChimeraError, match="static workspace") as e:
        run(ctx, ctx.search_device_noalloc, q, 10)
    assert e.value.code == capi.ERR_CAPACITY
    fit = int(re.search(r"at most (\d+) queries", str(e.value)).group(1))
    assert 1 <= fit < 16
    # the largest batch named in the message runs, one more does not
    want = run(ctx, ctx.search_device, q[:fit], 10)
    got = run(ctx, ctx.search_device_noalloc, q[:fit], 10)
    assert np.array_equal(got[0], want[0])
    with pytest.raises(capi.ChimeraError, match="static workspace"):
        run(ctx, ctx.search_device_noalloc, q[:fit + 1], 10)
    ctx.close()
