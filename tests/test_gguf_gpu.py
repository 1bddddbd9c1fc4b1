"""A MoE layer read from a GGUF file (include/osmos/model/gguf.h + libosmos_amd/gguf.py) and run on the MI355X: the
expert tensors llama.cpp names blk.N.ffn_{gate,up,down}_exps.weight (dims [cols, rows, n_exp], experts back to back)
are found by gguf_create, read in place, put on the device as they lie and handed to osmos_lane_layer - the oracle's
bits for the same bytes. (What the reference's tests do with real model files, e.g. tests/gpu/test_q8_gpu.hip:173-175's
experts of a real GGUF; no real model is on these machines, so the file is written here.)"""
import math

import numpy as np
import pytest

import gguf_writer as W
from libosmos_amd import synth
from test_moe_gpu import _lane_layer_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g():
    import torch  # noqa: F401
    from tests import gpu_util
    return gpu_util


@pytest.mark.parametrize("name,dim,ff", [("IQ3_XXS", 1024, 256), ("IQ2_XXS", 4096, 512)])
def test_layer_from_gguf(g, tmp_path, name, dim, ff):
    import torch
    from libosmos_amd.gguf import Model
    from libosmos_amd.layer import LaneLayer
    t = synth.ID[name]
    n_exp, k, n_tok = 6, 3, 5
    gate = [synth.iq_blocks(t, ff, dim, 10 + e) for e in range(n_exp)]
    up = [synth.iq_blocks(t, ff, dim, 20 + e) for e in range(n_exp)]
    down = [synth.iq_blocks(t, dim, ff, 30 + e) for e in range(n_exp)]
    tensors = [("blk.0.ffn_gate_exps.weight", t, [dim, ff, n_exp], np.concatenate(gate).tobytes(), None),
               ("blk.0.ffn_up_exps.weight", t, [dim, ff, n_exp], np.concatenate(up).tobytes(), None),
               ("blk.0.ffn_down_exps.weight", t, [ff, dim, n_exp], np.concatenate(down).tobytes(), None)]
    kv = [("general.architecture", W.STR, "qwen3moe"), ("qwen3moe.expert_count", W.U32, n_exp),
          ("qwen3moe.expert_used_count", W.U32, k)]
    path = tmp_path / "moe.gguf"
    path.write_bytes(W.model(tensors, kv)[0])
    print("gguf layer", name, dim, ff, flush=True)
    with Model(str(path)) as m:
        assert m.kv["qwen3moe.expert_count"] == n_exp and m.kv["qwen3moe.expert_used_count"] == k
        wg, tg, rows_g, cols_g = m.experts("blk.0.ffn_gate_exps.weight", torch)
        wu, _, _, _ = m.experts("blk.0.ffn_up_exps.weight", torch)
        wd, td, rows_d, cols_d = m.experts("blk.0.ffn_down_exps.weight", torch)
    assert (tg, td, rows_g, cols_g, rows_d, cols_d) == (t, t, ff, dim, dim, ff)
    assert wg.shape == (n_exp, ff * dim // 256 * synth.TYPES[t][2])
    L = LaneLayer(t, t, dim, ff, n_exp, k, wg, wu, wd)
    rng = np.random.default_rng(dim)
    x = rng.normal(0, 1, (n_tok, dim)).astype(np.float32)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    wts = rng.uniform(0.01, 0.3, (n_tok, k)).astype(np.float32)
    want = _lane_layer_oracle(t, x, ids, wts, gate, up, down, dim, ff, math.inf)
    out = torch.full((n_tok, dim), float("nan"), device="cuda")
    L.forward(g.dev(x), g.dev(ids), g.dev(wts), torch.zeros((n_tok, dim), device="cuda"), out)
    assert (g.bits(g.host(out)) == g.bits(want)).all()
