"""The allocation-free linear, vk_linear_run_into_noalloc_f32, against
vk_linear_run_into_f32 (the same plan, so the same bits) through the C ABI.

* two calls in a row on split-K plans, the second with fewer rows (the
  static scratch keeps the first call's partial sums: every slice the
  second call reads must be its own);
* a plain (unsplit, narrow-kernel) shape;
* capture into a HIP graph on a fresh runtime with no eager run first,
  where the allocating entry point must refuse (its work buffer cannot grow
  during capture), replayed three times with eager work in between;
* a plan whose partial sums exceed the scratch is refused with a clear
  error and enqueues nothing.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

vh = pytest.importorskip("vestra_hip")


def normals(rng, *shape, scale=1.0):
    return (scale * rng.standard_normal(shape)).astype(np.float32)


def make_linear(rt, rng, k, n, with_ls=False):
    ls = rng.uniform(0, 0.1, n).astype(np.float32) if with_ls else None
    return rt.prepare_linear_f32(k, n, normals(rng, k, n, scale=0.02), normals(rng, n, scale=0.02),
                                 ls)


@pytest.mark.parametrize("k,n,rows", [(3072, 768, (866, 433)), (768, 768, (866, 500))],
                         ids=["fc2-split6-then-3", "proj-split3-then-2"])
def test_two_calls_in_a_row_match_the_allocating_entry(rt, rng, k, n, rows):
    lin = make_linear(rt, rng, k, n, with_ls=True)
    for m in rows:  # the second call has fewer rows
        print(f"noalloc linear {m}x{k}->{n}", flush=True)
        x = rt.upload_f32(normals(rng, m, k))
        got, want = rt.alloc_f32(m * n), rt.alloc_f32(m * n)
        lin.run_into_noalloc(x, m, got)
        lin.run_into(x, m, want)
        assert np.array_equal(got.numpy(), want.numpy()), f"{m} rows"


def test_unsplit_and_narrow_shapes(rt, rng):
    for k, n, m in ((768, 3072, 866), (13, 8, 5)):
        lin = make_linear(rt, rng, k, n)
        x = rt.upload_f32(normals(rng, m, k))
        got, want = rt.alloc_f32(m * n), rt.alloc_f32(m * n)
        lin.run_into_noalloc(x, m, got)
        lin.run_into(x, m, want)
        assert np.array_equal(got.numpy(), want.numpy()), f"{m}x{k}->{n}"


def test_captures_without_an_eager_run(rng):
    import gc
    fresh = vh.Runtime(0)
    k, n, m = 3072, 768, 866
    lin = make_linear(fresh, rng, k, n)
    xh = normals(rng, m, k)
    x = fresh.upload_f32(xh)
    got = fresh.alloc_f32(m * n)
    fresh.synchronize()
    gc.disable()
    try:
        fresh.begin_capture()
        try:
            # the allocating form would have to grow its work buffer now
            with pytest.raises(vh.VestraError, match="before stream capture"):
                lin.run_into(x, m, got)
            lin.run_into_noalloc(x, m, got)
        finally:
            graph = fresh.end_capture()
    finally:
        gc.enable()
    want = fresh.alloc_f32(m * n)
    lin.run_into(x, m, want)  # eager now: the work buffer may grow
    expect = want.numpy()
    for r in range(3):
        got.write(np.zeros(m * n, np.float32))
        graph.launch()
        fresh.synchronize()
        assert np.array_equal(got.numpy(), expect), f"replay {r}"
        # eager work between replays, on other data
        lin.run_into(x, m, want)
    del graph, lin, x, got, want
    fresh.close()


def test_refuses_a_plan_beyond_the_scratch(rt, rng):
    # ViT-L's FC2 at 3,458 rows runs 8 split-K slices: 28 Mi floats
    k, n, m = 4096, 1024, 3458
    lin = make_linear(rt, rng, k, n)
    x = rt.upload_f32(normals(rng, m, k, scale=0.1))
    out = rt.upload_f32(np.full(m * n, 7.0, np.float32))
    with pytest.raises(vh.UnsupportedShape, match="scratch"):
        lin.run_into_noalloc(x, m, out)
    rt.synchronize()
    assert np.all(out.numpy() == 7.0)  # nothing was enqueued
