"""Parity of the per-layer decode steps with the CPU oracle.

fused_attention_step_w4a32 / _w8a32 restate src/quantization/fused_ops.rs:891-1062
and 718-888: QKV (+bias) -> RoPE with the position's cos / sin row -> k, v into
the caches at `offset` -> GQA attention over 0..offset -> O (+bias).
fused_transformer_layer_step_w4a32 restates src/quantization/fused_transformer.rs:16-376:
x += attention(RMSNorm(x)); x += down(silu(gate) * up)(RMSNorm(x)).  The oracle
side composes the oracle's pinned pieces (gemm_w4, gemv_w8, rope_apply,
attention, rms_norm, swiglu_mlp_w4).  Metric max|d| / max|ref|
(tests/parity/int4.rs:131-141); bar 2e-4 for the composed steps, as for the
decoder step.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from torchburn_amd import synth
import torchburn_amd as tb

pytestmark = pytest.mark.gpu

TOL = 2e-4
# W4A8 steps round every projection input to bytes, intermediates included: an
# element within ~1e-7 of a rounding boundary (f32 summation order) can land
# one byte over, a one-quantum step in what follows
A8_TOL = 3e-3


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def oracle_attention_step(x, qkv, o, kc, vc, cos_row, sin_row, offset, hq, hkv, hd, proj):
    """The reference step on the oracle's pieces; kc / vc [hkv, max, hd] updated in place."""
    y = proj(x, *qkv)
    q = y[: hq * hd].reshape(hq, hd)
    k = y[hq * hd: (hq + hkv) * hd].reshape(hkv, hd)
    v = y[(hq + hkv) * hd:].reshape(hkv, hd)
    q = np.stack([O.rope_apply(q[h], cos_row, sin_row) for h in range(hq)])
    k = np.stack([O.rope_apply(k[h], cos_row, sin_row) for h in range(hkv)])
    kc[:, offset] = k
    vc[:, offset] = v
    attn = O.attention(q, kc, vc, offset + 1).reshape(-1)
    return proj(attn, *o)


def w4proj(gs):
    return lambda x, w, s, b: O.gemm_w4(x.reshape(1, -1), w, s, b, group_size=gs)[0]


def w8proj(x, w, s, b):
    return O.gemv_w8(x.reshape(1, -1), w, s, b)[0]


def setup(g, H, hq, hkv, hd, max_seq, offset, bits, gs, theta):
    nq = (hq + 2 * hkv) * hd
    if bits == 4:
        qw, qs = synth.int4_weight(g, nq, H, gs)
        ow, os_ = synth.int4_weight(g, H, hq * hd, gs)
    else:
        qw, qs = synth.int8_weight(g, nq, H)
        ow, os_ = synth.int8_weight(g, H, hq * hd)
    qb = g.normal(0, 0.02, nq).astype(np.float32)
    ob = g.normal(0, 0.02, H).astype(np.float32)
    kc = np.zeros((1, hkv, max_seq, hd), np.float32)
    vc = np.zeros((1, hkv, max_seq, hd), np.float32)
    kc[:, :, :offset] = g.standard_normal((1, hkv, offset, hd), dtype=np.float32)
    vc[:, :, :offset] = g.standard_normal((1, hkv, offset, hd), dtype=np.float32)
    ct, st = O.rope_tables(max_seq, hd, theta)
    x = synth.activations(g, 1, H)
    return x, (qw, qs, qb), (ow, os_, ob), kc, vc, ct[offset], st[offset]


CASES = [
    # H, hq, hkv, hd, max_seq, offset, gs, theta
    (896, 14, 2, 64, 2112, 2048, 32, 1e6),      # Qwen2.5-0.5B shape, KV 2048
    (4096, 32, 8, 128, 4160, 4096, 32, 5e5),    # Llama-3-8B shape, KV 4096
    (512, 8, 8, 64, 80, 0, 64, 1e4),            # MHA, first position, group 64
    (1024, 16, 4, 64, 300, 200, 32, 1e4),       # ragged last tile
    # long caches: more 64-position tiles than the 128 attention blocks per KV
    # head, so blocks fold 2-3 tiles each (the merge reads 128 partials)
    (1024, 16, 4, 64, 16448, 12000, 32, 1e4),
    (2048, 16, 4, 128, 24640, 20000, 32, 5e5),
]


@pytest.mark.parametrize("H,hq,hkv,hd,max_seq,offset,gs,theta", CASES)
def test_attention_step_w4_matches_oracle(cuda, H, hq, hkv, hd, max_seq, offset, gs, theta):
    print(f"case fused_attention_step_w4a32 H={H} hq={hq} hkv={hkv} hd={hd} offset={offset}",
          flush=True)
    g = synth.rng(81, H, hq, hkv, offset)
    x, qkv, o, kc, vc, cr, sr = setup(g, H, hq, hkv, hd, max_seq, offset, 4, gs, theta)
    kc_ref, vc_ref = kc[0].copy(), vc[0].copy()
    ref = oracle_attention_step(x[0], qkv, o, kc_ref, vc_ref, cr, sr, offset, hq, hkv, hd,
                                w4proj(gs))
    kg, vg = T(kc, cuda), T(vc, cuda)
    out = tb.fused_attention_step_w4a32(T(x, cuda), *(T(a, cuda) for a in qkv),
                                        *(T(a, cuda) for a in o), kg, vg, T(cr, cuda),
                                        T(sr, cuda), offset, hq, hkv, hd, gs)
    torch.cuda.synchronize()
    err = rel(out.cpu().numpy()[0], ref)
    print(f"max rel err {err:.3g}", flush=True)
    assert err < TOL
    kn, vn = kg.cpu().numpy()[0], vg.cpu().numpy()[0]
    assert rel(kn[:, offset], kc_ref[:, offset]) < 1e-4
    assert rel(vn[:, offset], vc_ref[:, offset]) < 1e-4
    # every other cache position is untouched
    keep = np.ones(max_seq, bool)
    keep[offset] = False
    assert np.array_equal(kn[:, keep], kc[0][:, keep])
    assert np.array_equal(vn[:, keep], vc[0][:, keep])


@pytest.mark.parametrize("H,hq,hkv,hd,max_seq,offset", [(896, 14, 2, 64, 2112, 2048),
                                                        (4096, 32, 8, 128, 4160, 4096)])
def test_attention_step_w8_matches_oracle(cuda, H, hq, hkv, hd, max_seq, offset):
    print(f"case fused_attention_step_w8a32 H={H} hq={hq} offset={offset}", flush=True)
    g = synth.rng(82, H, hq, offset)
    x, qkv, o, kc, vc, cr, sr = setup(g, H, hq, hkv, hd, max_seq, offset, 8, 32, 1e6)
    kc_ref, vc_ref = kc[0].copy(), vc[0].copy()
    ref = oracle_attention_step(x[0], qkv, o, kc_ref, vc_ref, cr, sr, offset, hq, hkv, hd,
                                w8proj)
    kg, vg = T(kc, cuda), T(vc, cuda)
    out = tb.fused_attention_step_w8a32(T(x, cuda), *(T(a, cuda) for a in qkv),
                                        *(T(a, cuda) for a in o), kg, vg, T(cr, cuda),
                                        T(sr, cuda), offset, hq, hkv, hd)
    torch.cuda.synchronize()
    err = rel(out.cpu().numpy()[0], ref)
    print(f"max rel err {err:.3g}", flush=True)
    assert err < TOL
    assert rel(kg.cpu().numpy()[0][:, offset], kc_ref[:, offset]) < 1e-4


@pytest.mark.parametrize("H,I,hq,hkv,hd,max_seq,offset,eps", [
    (896, 4864, 14, 2, 64, 2112, 2048, 1e-6),
    (4096, 14336, 32, 8, 128, 4160, 4096, 1e-5),
])
def test_transformer_layer_step_matches_oracle(cuda, H, I, hq, hkv, hd, max_seq, offset, eps):
    print(f"case fused_transformer_layer_step_w4a32 H={H} I={I} offset={offset}", flush=True)
    g = synth.rng(83, H, I)
    x, qkv, o, kc, vc, cr, sr = setup(g, H, hq, hkv, hd, max_seq, offset, 4, 32, 1e6)
    in_w = (1.0 + g.normal(0, 0.1, H)).astype(np.float32)
    post_w = (1.0 + g.normal(0, 0.1, H)).astype(np.float32)
    gw, gsc = synth.int4_weight(g, I, H, 32)
    uw, usc = synth.int4_weight(g, I, H, 32)
    dw, dsc = synth.int4_weight(g, H, I, 32)
    gb = g.normal(0, 0.02, I).astype(np.float32)
    db = g.normal(0, 0.02, H).astype(np.float32)
    # oracle
    kc_ref, vc_ref = kc[0].copy(), vc[0].copy()
    xr = x[0].copy()
    xn = O.rms_norm(xr, in_w, eps)
    xr = xr + oracle_attention_step(xn, qkv, o, kc_ref, vc_ref, cr, sr, offset, hq, hkv, hd,
                                    w4proj(32))
    xn = O.rms_norm(xr, post_w, eps)
    xr = xr + O.swiglu_mlp_w4(xn.reshape(1, -1), gw, gsc, uw, usc, dw, dsc, gb=gb, db=db,
                              group_size=32)[0]
    # GPU, x updated in place
    xg = T(x, cuda)
    kg, vg = T(kc, cuda), T(vc, cuda)
    tb.fused_transformer_layer_step_w4a32(
        xg, T(in_w, cuda), *(T(a, cuda) for a in qkv), *(T(a, cuda) for a in o),
        T(post_w, cuda), T(gw, cuda), T(gsc, cuda), T(gb, cuda), T(uw, cuda), T(usc, cuda), None,
        T(dw, cuda), T(dsc, cuda), T(db, cuda), kg, vg, T(cr, cuda), T(sr, cuda), offset, hq,
        hkv, hd, 32, eps)
    torch.cuda.synchronize()
    err = rel(xg.cpu().numpy()[0], xr)
    print(f"max rel err {err:.3g}", flush=True)
    assert err < TOL
    assert rel(kg.cpu().numpy()[0][:, offset], kc_ref[:, offset]) < 1e-4


def a8proj(x, w, s, b):
    return O.gemm_w4a8_g64(x.reshape(1, -1), w, s, b)[0]


@pytest.mark.parametrize("H,I,hq,hkv,hd,max_seq,offset,eps", [
    (896, 4864, 14, 2, 64, 2112, 2048, 1e-6),
    (4096, 14336, 32, 8, 128, 4160, 4096, 1e-5),
])
def test_layer_steps_vnni_semantics(cuda, H, I, hq, hkv, hd, max_seq, offset, eps):
    """Group 64 under W4A8 semantics (tb_set_vnni_semantics): every projection of
    the attention step and the layer step contracts its input's bytes, as on the
    reference's AVX-512 VNNI hosts (gemv.rs:1559-1563; the SwiGLU pair
    fused_transformer.rs:299); against the oracle's W4A8 pieces, and far from
    the exact steps."""
    print(f"case layer steps vnni H={H} I={I} offset={offset}", flush=True)
    g = synth.rng(86, H, I)
    x, qkv, o, kc, vc, cr, sr = setup(g, H, hq, hkv, hd, max_seq, offset, 4, 64, 1e6)
    in_w = (1.0 + g.normal(0, 0.1, H)).astype(np.float32)
    post_w = (1.0 + g.normal(0, 0.1, H)).astype(np.float32)
    gw, gsc = synth.int4_weight(g, I, H, 64)
    uw, usc = synth.int4_weight(g, I, H, 64)
    dw, dsc = synth.int4_weight(g, H, I, 64)
    gb = g.normal(0, 0.02, I).astype(np.float32)
    db = g.normal(0, 0.02, H).astype(np.float32)
    # oracle: the attention step alone, then the layer step
    ka, va = kc[0].copy(), vc[0].copy()
    ref_att = oracle_attention_step(x[0], qkv, o, ka, va, cr, sr, offset, hq, hkv, hd, a8proj)
    exact_att = oracle_attention_step(x[0], qkv, o, kc[0].copy(), vc[0].copy(), cr, sr, offset,
                                      hq, hkv, hd, w4proj(64))
    kr, vr = kc[0].copy(), vc[0].copy()
    xr = x[0].copy()
    xn = O.rms_norm(xr, in_w, eps)
    xr = xr + oracle_attention_step(xn, qkv, o, kr, vr, cr, sr, offset, hq, hkv, hd, a8proj)
    xn = O.rms_norm(xr, post_w, eps)
    xr = xr + O.swiglu_mlp_w4a8(xn.reshape(1, -1), gw, gsc, uw, usc, dw, dsc, gb=gb, db=db)[0]
    prev = tb.set_vnni_semantics(True)
    try:
        kg, vg = T(kc, cuda), T(vc, cuda)
        out = tb.fused_attention_step_w4a32(T(x, cuda), *(T(a, cuda) for a in qkv),
                                            *(T(a, cuda) for a in o), kg, vg, T(cr, cuda),
                                            T(sr, cuda), offset, hq, hkv, hd, 64)
        xg = T(x, cuda)
        kl, vl = T(kc, cuda), T(vc, cuda)
        tb.fused_transformer_layer_step_w4a32(
            xg, T(in_w, cuda), *(T(a, cuda) for a in qkv), *(T(a, cuda) for a in o),
            T(post_w, cuda), T(gw, cuda), T(gsc, cuda), T(gb, cuda), T(uw, cuda), T(usc, cuda),
            None, T(dw, cuda), T(dsc, cuda), T(db, cuda), kl, vl, T(cr, cuda), T(sr, cuda),
            offset, hq, hkv, hd, 64, eps)
        torch.cuda.synchronize()
    finally:
        tb.set_vnni_semantics(prev)
    e1 = rel(out.cpu().numpy()[0], ref_att)
    e2 = rel(xg.cpu().numpy()[0], xr)
    ex = rel(out.cpu().numpy()[0], exact_att)
    print(f"max rel err attention step {e1:.3g}, layer step {e2:.3g}; the W4A32 attention "
          f"step is off by {ex:.3g}", flush=True)
    assert e1 < A8_TOL and e2 < A8_TOL
    assert ex > 5 * max(e1, 1e-6)
    assert rel(kg.cpu().numpy()[0][:, offset], ka[:, offset]) < 1e-4


def test_layer_step_on_cpu_tensors_mutates_in_place(cuda):
    """CPU tensors in, as the reference takes them: the caches and x are updated in
    place and the result equals the device-tensor call."""
    print("case layer steps on host tensors", flush=True)
    H, hq, hkv, hd, max_seq, offset = 512, 8, 2, 64, 96, 40
    g = synth.rng(84)
    x, qkv, o, kc, vc, cr, sr = setup(g, H, hq, hkv, hd, max_seq, offset, 4, 32, 1e4)
    kd, vd = T(kc, cuda), T(vc, cuda)
    ref = tb.fused_attention_step_w4a32(T(x, cuda), *(T(a, cuda) for a in qkv),
                                        *(T(a, cuda) for a in o), kd, vd, T(cr, cuda),
                                        T(sr, cuda), offset, hq, hkv, hd, 32).cpu()
    kh, vh = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    out = tb.fused_attention_step_w4a32(torch.from_numpy(x), *(torch.from_numpy(a) for a in qkv),
                                        *(torch.from_numpy(a) for a in o), kh, vh,
                                        torch.from_numpy(cr), torch.from_numpy(sr), offset, hq,
                                        hkv, hd, 32)
    assert out.device.type == "cpu"
    assert torch.equal(out, ref)
    assert torch.equal(kh, kd.cpu()) and torch.equal(vh, vd.cpu())


def test_layer_step_errors(cuda):
    H, hq, hkv, hd, max_seq = 512, 8, 2, 64, 64
    g = synth.rng(85)
    x, qkv, o, kc, vc, cr, sr = setup(g, H, hq, hkv, hd, max_seq, 10, 4, 32, 1e4)
    args = lambda off, heads, kvh: (T(x, cuda), *(T(a, cuda) for a in qkv),
                                    *(T(a, cuda) for a in o), T(kc, cuda), T(vc, cuda),
                                    T(cr, cuda), T(sr, cuda), off, heads, kvh, hd, 32)
    with pytest.raises(tb.UnsupportedOpError, match="offset"):
        tb.fused_attention_step_w4a32(*args(max_seq, hq, hkv))
    with pytest.raises(tb.UnsupportedOpError):
        tb.fused_attention_step_w4a32(*args(10, hq, 3))
    # head_dim outside {64, 128} is rejected before any kernel writes the caches
    # (16 heads of 32 and 4 KV heads: the same QKV rows and O width as 8 x 64 / 2 x 64)
    kc32 = T(np.zeros((1, 2 * hkv, max_seq, 32), np.float32), cuda)
    with pytest.raises(tb.UnsupportedOpError, match="head_dim"):
        tb.fused_attention_step_w4a32(T(x, cuda), *(T(a, cuda) for a in qkv),
                                      *(T(a, cuda) for a in o), kc32, kc32.clone(),
                                      T(cr[:32], cuda), T(sr[:32], cuda), 10, 2 * hq, 2 * hkv,
                                      32, 32)
    assert not kc32.any()
