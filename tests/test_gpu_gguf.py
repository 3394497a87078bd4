"""Expert banks loaded from a GGUF file drive the kernels: the layer's
tensors are written to a file in the GGUF layout (separate and fused
gate_up, with and without biases), uploaded by `gguf.upload_layer`, routed
through `moe_route_ptrs` with the file's bank, and the pair / down outputs
must equal, bit for bit, those of the same weights uploaded directly, and
match the oracle."""
import numpy as np
import pytest
import torch

import oracle
from pulsar_amd import gguf as G
from pulsar_amd import kernels as K
from pulsar_amd.formats import ACT_SILU, ACT_SWIGLU_OAI, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K, QUANT_Q6_K
from tests.gpu_util import down, up, up_f32, zeros_f32
from tests.test_gpu_moe import Layer, down_bound, pair_bound

pytestmark = pytest.mark.gpu

TYPE_OF = {QUANT_Q4_K: G.TensorType.Q4_K, QUANT_Q6_K: G.TensorType.Q6_K, QUANT_Q2_K: G.TensorType.Q2_K,
           QUANT_MXFP4: G.TensorType.MXFP4}


def _write(path, L: Layer, fused: bool):
    E, ff, hid = L.E, L.ffn, L.hidden
    t = []
    if fused:
        gu = np.concatenate([L.g, L.u], axis=1)  # [E][2 ff][row bytes]: gate rows, then up rows
        t.append(("blk.0.ffn_gate_up_exps.weight", (hid, 2 * ff, E), TYPE_OF[L.gq], gu.tobytes()))
    else:
        t.append(("blk.0.ffn_gate_exps.weight", (hid, ff, E), TYPE_OF[L.gq], L.g.tobytes()))
        t.append(("blk.0.ffn_up_exps.weight", (hid, ff, E), TYPE_OF[L.gq], L.u.tobytes()))
    t.append(("blk.0.ffn_down_exps.weight", (ff, hid, E), TYPE_OF[L.dq], L.d.tobytes()))
    if L.gb is not None:
        t += [("blk.0.ffn_gate_exps.bias", (ff, E), G.TensorType.F32, L.gb.tobytes()),
              ("blk.0.ffn_up_exps.bias", (ff, E), G.TensorType.F32, L.ub.tobytes()),
              ("blk.0.ffn_down_exps.bias", (hid, E), G.TensorType.F32, L.db.tobytes())]
    G.write_gguf(path, {"general.architecture": "test", "test.expert_count": E}, t, alignment=64)


@pytest.mark.parametrize("gq,dq,fused,biases,act", [
    (QUANT_Q4_K, QUANT_Q6_K, False, False, ACT_SILU),
    (QUANT_Q4_K, QUANT_Q2_K, True, False, ACT_SILU),
    (QUANT_MXFP4, QUANT_MXFP4, False, True, ACT_SWIGLU_OAI),
])
def test_gguf_bank_drives_kernels(dev, tmp_path, gq, dq, fused, biases, act):
    hidden, ffn = (576, 320) if gq == QUANT_MXFP4 else (512, 256)
    L = Layer(gq, dq, hidden=hidden, ffn=ffn, E=5, n_used=3, n_tok=4, biases=biases, null_slots=(4,))
    p = tmp_path / "layer.gguf"
    _write(p, L, fused)
    g = G.Gguf.open(p)
    lx, bank, keep = G.upload_layer(p, g, 0, dev)
    assert (lx.fused_up_off != 0) == fused and lx.gate.quant == gq and lx.down.quant == dq
    n_slots, f32 = L.n_used, dict(dtype=torch.float32, device=dev)
    sel = up(L.sel.astype(np.int32))
    ptrs = torch.zeros(L.n_tok * n_slots * 48, dtype=torch.uint8, device=dev)
    slot_w = zeros_f32((L.n_tok, n_slots))
    K.moe_route_ptrs(ptrs, slot_w, sel, up_f32(L.w), bank, L.E, None, L.n_tok, n_slots)
    hptrs, dptrs = L.ptrs()  # the same weights uploaded directly
    xq = oracle.quantize_q8_k(L.x)
    mids = []
    for pp in (ptrs, dptrs):
        mid = zeros_f32((L.n_tok * n_slots, ffn))
        K.moe_pair_swiglu(mid, pp, up_f32(L.w), up(xq), hidden, ffn, n_slots, L.n_tok, lx.gate.row_bytes, gq, act)
        mids.append(down(mid))
    assert np.array_equal(mids[0], mids[1])
    want_mid = oracle.moe_pair_swiglu(hptrs, L.w, xq, hidden, ffn, n_slots, L.n_tok, L.grb, gq, act)
    bound = pair_bound(L, xq, act) + 4e-7 * np.abs(want_mid) + 1e-30
    assert (np.abs(mids[0].astype(np.float64) - want_mid) <= bound).all()
    midq = oracle.quantize_q8_k(want_mid)
    outs = []
    for pp in (ptrs, dptrs):
        out = torch.zeros((L.n_tok, hidden), **f32)
        K.moe_down(out, pp, up(midq), ffn, hidden, n_slots, L.n_tok, lx.down.row_bytes, dq)
        if biases:
            K.moe_down_bias(out, pp, up_f32(L.w), hidden, n_slots, L.n_tok)
        outs.append(down(out))
    assert np.array_equal(outs[0], outs[1])
    if not biases:
        want = oracle.moe_down(hptrs, midq, ffn, hidden, n_slots, L.n_tok, L.drb, dq)
        assert (np.abs(outs[0].astype(np.float64) - want) <= down_bound(L, midq)).all()
    del keep
