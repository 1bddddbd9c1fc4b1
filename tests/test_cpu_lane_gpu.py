"""The lane's CPU hand-off end to end on the MI355X (reference src/run/hip_lane.c:115-222): a step's tables built on
the device (osmos_lane_tables), some experts left to the host pool (cpu_lane_submit: their rows into mapped host
memory, the flag posted), the others run on the GPU through the drop-in kernels (q8_round, q8_gate_up, q8_round,
q8_group_tok); the stream held on the flag (ops_wait), the host's rows taken beside the GPU's (ops_copy_rows), each
token's rows summed in ascending expert id (ops_gather_sum_add) - the bits of the all-GPU layer (osmos_lane_layer)."""
import ctypes

import numpy as np
import pytest

from libosmos_amd import capi, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


@pytest.mark.parametrize("name,dim,ff", [("IQ3_XXS", 1024, 256), ("IQ2_XXS", 4096, 512), ("Q4_K", 2048, 512)])
def test_handoff_layer_bits(g, name, dim, ff):
    import torch
    from libosmos_amd.layer import LaneLayer
    t = synth.ID[name]
    n_exp, k, n_tok, lim = 12, 4, 5, 2.0
    mk = synth.iq_blocks if name.startswith("IQ") else synth.random_blocks
    G = np.stack([mk(t, ff, dim, 300 + e) for e in range(n_exp)])
    U = np.stack([mk(t, ff, dim, 400 + e) for e in range(n_exp)])
    D = np.stack([mk(t, dim, ff, 500 + e) for e in range(n_exp)])
    rng = np.random.default_rng(dim)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.uniform(0.05, 0.4, (n_tok, k)).astype(np.float32)
    Gd, Ud, Dd = g.dev(G).reshape(n_exp, -1), g.dev(U).reshape(n_exp, -1), g.dev(D).reshape(n_exp, -1)
    add = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    # the all-GPU layer
    layer = LaneLayer(t, t, dim, ff, n_exp, k, Gd, Ud, Dd, lim=lim)
    want = torch.full((n_tok, dim), float("nan"), device="cuda")
    layer.forward(g.dev(x), g.dev(ids), g.dev(w), g.dev(add), want)
    want = g.host(want)
    # the step's tables on the device
    L = capi.lib()
    P = n_tok * k
    i32 = lambda: torch.zeros(P, dtype=torch.int32, device="cuda")  # noqa: E731
    tok, pair, cnt, xrow, order = i32(), i32(), i32(), i32(), i32()
    wg, wu, wd = (torch.zeros(P, dtype=torch.int64, device="cuda") for _ in range(3))
    base = (ctypes.c_void_p * 3)(Gd.data_ptr(), Ud.data_ptr(), Dd.data_ptr())
    nbytes = (ctypes.c_uint64 * 3)(Gd[0].numel(), Ud[0].numel(), Dd[0].numel())
    ids_d = g.dev(ids)
    print("hand-off", name, dim, ff, flush=True)
    assert L.osmos_lane_tables(g.a(ids_d), n_tok, k, n_exp, base, nbytes, g.a(tok), g.a(pair), g.a(cnt), g.a(xrow),
                               g.a(wg), g.a(wu), g.a(wd), g.a(order), None)
    tok_h, pair_h, cnt_h, xrow_h = (g.host(a_) for a_ in (tok, pair, cnt, xrow))
    live = [e for e in range(P) if cnt_h[e] > 0]
    ex = {e: int(ids.reshape(-1)[pair_h[xrow_h[e]]]) for e in live}
    on_cpu = [e for e in live if ex[e] % 3 == 0]
    assert on_cpu and len(on_cpu) < len(live)
    # the host's experts: a job over the pair rows (x by token, the weight by pick), their outputs at their own rows
    x_pairs = np.ascontiguousarray(x[tok_h])
    scale = np.ascontiguousarray(w.reshape(-1)[pair_h])
    es = (capi.CpuLaneExpert * len(on_cpu))(*[capi.CpuLaneExpert(G[ex[e]].ctypes.data, U[ex[e]].ctypes.data,
                                                                 D[ex[e]].ctypes.data, int(xrow_h[e]), int(cnt_h[e]))
                                              for e in on_cpu])
    y_host = torch.full((P, dim), float("nan"), pin_memory=True)  # (host memory the GPU maps)
    seq = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    value = 11
    job = capi.CpuLaneJob(t, t, dim, ff, lim, x_pairs.ctypes.data, scale.ctypes.data, P, es, len(on_cpu),
                          y_host.data_ptr(), seq.data_ptr(), value)
    pool = L.cpu_lane_create(4, None, P, dim, ff)
    assert pool
    try:
        cnt_gpu = cnt_h.copy()
        cnt_gpu[on_cpu] = 0  # (the GPU skips an entry of no rows)
        cnt_g = g.dev(cnt_gpu)
        cpu_rows = g.dev(np.concatenate([np.arange(xrow_h[e], xrow_h[e] + cnt_h[e]) for e in on_cpu]).astype(np.int32))
        n_cpu = int(cpu_rows.numel())
        xq = torch.zeros(n_tok, dim, dtype=torch.int8, device="cuda")
        xd = torch.zeros(n_tok, dim // 32, device="cuda")
        h = torch.zeros(P, ff, device="cuda")
        hq = torch.zeros(P, ff, dtype=torch.int8, device="cuda")
        hd = torch.zeros(P, ff // 32, device="cuda")
        ye = torch.full((P, dim), float("nan"), device="cuda")
        out = torch.full((n_tok, dim), float("nan"), device="cuda")
        max_cnt = int(cnt_h.max())
        s = torch.cuda.Stream()
        xg, wf, addg = g.dev(x), g.dev(w.reshape(-1)), g.dev(add)
        assert L.cpu_lane_submit(pool, ctypes.byref(job))  # the host's experts start now, beside the GPU's
        ok = (L.q8_round(g.a(xg), n_tok, dim, dim, g.a(xq), g.a(xd), s.cuda_stream) and
              L.q8_gate_up(t, g.a(wg), g.a(wu), g.a(cnt_g), g.a(xrow), g.a(tok), g.a(pair), P, max_cnt, ff, dim,
                           g.a(xq), g.a(xd), g.a(wf), lim, g.a(h), ff, s.cuda_stream) and
              L.q8_round(g.a(h), P, ff, ff, g.a(hq), g.a(hd), s.cuda_stream) and
              L.q8_group_tok(t, g.a(wd), g.a(cnt_g), g.a(xrow), None, P, max_cnt, dim, ff, g.a(hq), g.a(hd), g.a(ye),
                             dim, s.cuda_stream) and
              L.ops_wait(capi.addr(seq), value, s.cuda_stream) and
              L.ops_copy_rows(g.a(ye), capi.addr(y_host), g.a(cpu_rows), n_cpu, dim, s.cuda_stream) and
              L.ops_gather_sum_add(g.a(out), g.a(ye), g.a(order), k, n_tok, dim, g.a(addg), s.cuda_stream))
        assert ok
        assert L.cpu_lane_wait(pool)
        s.synchronize()
        got = g.host(out)
    finally:
        seq.fill_(value)  # (the stream's wait always ends)
        torch.cuda.synchronize()
        L.cpu_lane_destroy(pool)
    assert (g.bits(got) == g.bits(want)).all()
