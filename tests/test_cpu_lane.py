"""The lane's CPU half (include/osmos/cpu/lane.h: cpu_lane_create / submit / wait / destroy) on the host: a job's rows
the reference CPU lane's bits (the pinned oracle's orc_lane_layer, itself checked against the reference's compiled
src/cpu/lane.c phases) for the lane types at 16 and 32 logical lanes, whatever the pool's thread count; the flag posted
with the job's value; refusals with nothing queued. (reference test: tests/test_cpu_lane.c)"""
import ctypes
import math

import numpy as np
import pytest

from libosmos_amd import capi, synth
from oracle import orc

TYPES = ["IQ3_XXS", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ1_S", "IQ1_M", "Q2_K", "Q4_0", "Q4_K", "Q3_K"]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def make_job(t_gu, t_dn, dim, ff, n_e, cnt, seed, lim=math.inf):
    mk = lambda t: synth.iq_blocks if synth.TYPES[t][0].startswith("IQ") else synth.random_blocks  # noqa: E731
    rng = np.random.default_rng(seed)
    gate = [mk(t_gu)(t_gu, ff, dim, seed + 10 + e) for e in range(n_e)]
    up = [mk(t_gu)(t_gu, ff, dim, seed + 40 + e) for e in range(n_e)]
    down = [mk(t_dn)(t_dn, dim, ff, seed + 70 + e) for e in range(n_e)]
    n_rows = int(sum(cnt))
    x = rng.normal(0, 1, (n_rows, dim)).astype(np.float32)
    scale = rng.uniform(0.05, 0.5, n_rows).astype(np.float32)
    row0 = np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.uint32)
    return gate, up, down, x, scale, row0, np.array(cnt, np.uint32)


def oracle_rows(t_gu, t_dn, dim, ff, lim, gate, up, down, x, scale, row0, cnt):
    P = ctypes.c_void_p
    tab = lambda ms: (P * len(ms))(*[m.ctypes.data for m in ms])  # noqa: E731
    y = np.zeros((x.shape[0], dim), np.float32)
    assert orc.orc().orc_lane_layer(t_gu, t_dn, dim, ff, lim, orc.ptr(x), orc.ptr(scale), x.shape[0], tab(gate),
                                    tab(up), tab(down), orc.ptr(row0), orc.ptr(cnt), len(cnt), orc.ptr(y))
    return y


def run_pool(threads, t_gu, t_dn, dim, ff, lim, gate, up, down, x, scale, row0, cnt, value=7):
    L = capi.lib()
    pool = L.cpu_lane_create(threads, None, x.shape[0], dim, ff)
    assert pool
    try:
        es = (capi.CpuLaneExpert * len(cnt))(*[capi.CpuLaneExpert(gate[e].ctypes.data, up[e].ctypes.data,
                                                                  down[e].ctypes.data, int(row0[e]), int(cnt[e]))
                                               for e in range(len(cnt))])
        y = np.full((x.shape[0], dim), np.nan, np.float32)
        seq = np.zeros(1, np.uint32)
        job = capi.CpuLaneJob(t_gu, t_dn, dim, ff, lim, x.ctypes.data, scale.ctypes.data, x.shape[0], es, len(cnt),
                              y.ctypes.data, seq.ctypes.data, value)
        assert L.cpu_lane_submit(pool, ctypes.byref(job))
        assert L.cpu_lane_wait(pool)
        assert int(seq[0]) == value
        return y
    finally:
        L.cpu_lane_destroy(pool)


@pytest.mark.parametrize("name", TYPES)
def test_cpu_lane_job_bits(name):
    t = synth.ID[name]
    for dim, ff, threads in ((512, 256, 3), (4096, 512, 5)):  # (16 lanes; 32 lanes on gate / up)
        args = make_job(t, t, dim, ff, 4, [2, 1, 3, 1], 100 + dim)
        want = oracle_rows(t, t, dim, ff, 1.5, *args)
        got = run_pool(threads, t, t, dim, ff, 1.5, *args)
        assert (bits(got) == bits(want)).all(), (name, dim)


def test_cpu_lane_split_and_types():
    """one thread and 8 threads the same bits; gate/up and down of different types; an unclamped activation"""
    tg, td = synth.ID["IQ2_XXS"], synth.ID["IQ3_XXS"]
    args = make_job(tg, td, 1024, 512, 5, [1, 4, 2, 2, 3], 7)
    want = oracle_rows(tg, td, 1024, 512, math.inf, *args)
    for threads in (1, 8):
        got = run_pool(threads, tg, td, 1024, 512, math.inf, *args)
        assert (bits(got) == bits(want)).all(), threads


def test_cpu_lane_refusals():
    L = capi.lib()
    assert not L.cpu_lane_create(0, None, 4, 512, 256)
    assert not L.cpu_lane_create(65, None, 4, 512, 256)
    assert not L.cpu_lane_create(2, None, 4, 500, 256)  # dim not whole 256s
    pool = L.cpu_lane_create(2, None, 4, 512, 256)
    assert pool
    try:
        t = synth.ID["IQ3_XXS"]
        gate, up, down, x, scale, row0, cnt = make_job(t, t, 512, 256, 2, [2, 2], 1)
        es = (capi.CpuLaneExpert * 2)(*[capi.CpuLaneExpert(gate[e].ctypes.data, up[e].ctypes.data, down[e].ctypes.data,
                                                           int(row0[e]), int(cnt[e])) for e in range(2)])
        y = np.zeros((4, 512), np.float32)
        seq = np.full(1, 99, np.uint32)
        bad = [capi.CpuLaneJob(synth.ID["Q8_0"], t, 512, 256, 1.0, x.ctypes.data, scale.ctypes.data, 4, es, 2,
                               y.ctypes.data, seq.ctypes.data, 3),  # not a lane type
               capi.CpuLaneJob(t, t, 1024, 256, 1.0, x.ctypes.data, scale.ctypes.data, 4, es, 2, y.ctypes.data,
                               seq.ctypes.data, 3),  # dim not the pool's
               capi.CpuLaneJob(t, t, 512, 256, 1.0, x.ctypes.data, scale.ctypes.data, 5, es, 2, y.ctypes.data,
                               seq.ctypes.data, 3),  # rows past the pool's
               capi.CpuLaneJob(t, t, 512, 256, 1.0, x.ctypes.data, scale.ctypes.data, 3, es, 2, y.ctypes.data,
                               seq.ctypes.data, 3)]  # an expert's rows past the job's
        for j in bad:
            assert not L.cpu_lane_submit(pool, ctypes.byref(j))
        assert int(seq[0]) == 99  # nothing queued, the flag untouched
        assert L.cpu_lane_wait(pool)
    finally:
        L.cpu_lane_destroy(pool)


def test_cpu_lane_pinned_and_repeated():
    """workers pinned to given CPUs (a CPU that cannot be taken refuses the pool); one pool, several jobs in a row,
    each flag posted with its own value and the oracle's bits; more workers than rows"""
    import os
    L = capi.lib()
    assert not L.cpu_lane_create(2, (ctypes.c_int * 2)(0, -1), 4, 512, 256)
    cpus = sorted(os.sched_getaffinity(0))[:3]
    pool = L.cpu_lane_create(len(cpus), (ctypes.c_int * len(cpus))(*cpus), 8, 512, 256)
    assert pool
    try:
        t = synth.ID["IQ3_XXS"]
        for rep, cnt in enumerate(([1], [2, 1, 3], [1, 1])):
            gate, up, down, x, scale, row0, cn = make_job(t, t, 512, 256, len(cnt), cnt, 50 + rep)
            want = oracle_rows(t, t, 512, 256, 2.0, gate, up, down, x, scale, row0, cn)
            es = (capi.CpuLaneExpert * len(cnt))(*[capi.CpuLaneExpert(gate[e].ctypes.data, up[e].ctypes.data,
                                                                      down[e].ctypes.data, int(row0[e]), int(cn[e]))
                                                   for e in range(len(cnt))])
            y = np.full((x.shape[0], 512), np.nan, np.float32)
            seq = np.zeros(1, np.uint32)
            job = capi.CpuLaneJob(t, t, 512, 256, 2.0, x.ctypes.data, scale.ctypes.data, x.shape[0], es, len(cnt),
                                  y.ctypes.data, seq.ctypes.data, 100 + rep)
            assert L.cpu_lane_submit(pool, ctypes.byref(job))
            assert L.cpu_lane_wait(pool)
            assert int(seq[0]) == 100 + rep
            assert (bits(y) == bits(want)).all(), rep
    finally:
        L.cpu_lane_destroy(pool)
