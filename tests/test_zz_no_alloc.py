"""chimera_search_device_noalloc (the search on the library's static device
workspace) against chimera_search_device through the C ABI: identical ids,
scores and counts on two calls in a row, the second with a smaller batch
(the static workspace keeps the first call's contents), in both scoring
modes; a batch beyond the static workspace is rejected with a capacity
error."""
import numpy as np
import pytest

from chimera_amd import capi

pytestmark = pytest.mark.gpu


def run(ctx, fn, queries, k):
    nq = queries.shape[0]
    d_q = ctx.to_device(queries)
    d_ids = ctx.empty((nq, k), np.int64)
    d_sc = ctx.empty((nq, k), np.float32)
    d_cnt = ctx.empty((nq,), np.int32)
    try:
        fn(d_q, nq, k, d_ids, d_sc, d_cnt)
        ctx.synchronize()
        return d_ids.numpy(), d_sc.numpy(), d_cnt.numpy()
    finally:
        for a in (d_q, d_ids, d_sc, d_cnt):
            a.free()


@pytest.mark.parametrize("exact", [False, True], ids=["mfma", "exact"])
def test_noalloc_search_equals_search_device(small_index, small_workload, exact):
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=exact)
    print(f"no-alloc search: small index, exact={exact}, batches of 6 then 3 queries", flush=True)
    for nq, k in ((6, 50), (3, 20)):
        q = np.ascontiguousarray(small_workload.queries[16 - nq:], np.float32) if nq == 3 else \
            np.ascontiguousarray(small_workload.queries[:nq], np.float32)
        want = run(ctx, ctx.search_device, q, k)
        got = run(ctx, ctx.search_device_noalloc, q, k)
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
    ctx.close()
