"""Writes tests/golden/ref_vectors.npz: input/output vectors of the
reference's own CPU oracles for the hot path, produced by oracle/_ref
(the reference's oracle sources compiled where they lie, see oracle/Makefile)
on small seeded inputs.  Run in a container that has the reference checkout:

    make -C oracle ref && python tests/golden/make_golden.py

The fixtures pin the C restatement in oracle/pih_oracle.c to the reference
without needing the reference at test time (tests/test_oracle_golden.py).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from pih_amd import synth  # noqa: E402


def _p(a):
    return a.ctypes.data_as(oracle.P)


def main():
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref not built (make -C oracle ref needs /root/reference)")
    out = {}

    # e4m3 encode of a seeded spread of values incl. ties and edges
    vals = np.concatenate([
        (synth.normal(11, 2000) * 40).astype(np.float32),
        np.array([0.0, -0.0, 1.0, 1.0625, 1.1875, 448.0, -448.0, 2 ** -9, 2 ** -10, 3 * 2 ** -11,
                  0.0009765625, 240.0, 232.0, 1.0 / 3.0], np.float32)])
    vals = np.clip(vals, -448, 448).astype(np.float32)
    codes = np.empty(vals.size, np.uint8)
    b = oracle.C.c_uint8()
    for i, v in enumerate(vals):
        assert R.pr_e4m3_encode(float(v), oracle.C.byref(b)) == 0
        codes[i] = b.value
    out["e4m3_in"], out["e4m3_codes"] = vals, codes

    # FP8 activation quant (UE8M0)
    x = (synth.normal(12, 4 * 512) * np.repeat([1e-3, 1.0, 30.0, 1e3], 512)).astype(np.float32).reshape(4, 512)
    x[1, 128:256] = 0.0
    q = np.empty((4, 512), np.uint8)
    s = np.empty((4, 4), np.uint8)
    assert R.pr_fp8_quant(_p(x), 4, 512, _p(q), _p(s)) == 0
    out["quant_x"], out["quant_codes"], out["quant_scales"] = x, q, s

    # FP8 block GEMM
    m, n, k = 3, 128, 384
    a = synth.e4m3_encode((synth.normal(13, m * k) * 50).clip(-448, 448).astype(np.float32)).reshape(m, k)
    w = synth.e4m3_encode((synth.normal(14, n * k) * 50).clip(-448, 448).astype(np.float32)).reshape(n, k)
    sa = (120 + synth.splitmix64(15, m * 3) % np.uint64(8)).astype(np.uint8).reshape(m, 3)
    sw = (118 + synth.splitmix64(16, 1 * 3) % np.uint64(8)).astype(np.uint8).reshape(1, 3)
    o = np.empty((m, n), np.float32)
    assert R.pr_fp8_gemm(_p(a), _p(sa), _p(w), _p(sw), m, n, k, _p(o)) == 0
    out.update(fp8_a=a, fp8_sa=sa, fp8_w=w, fp8_sw=sw, fp8_out=o)

    # FP4 x FP8 GEMM
    m, n, k = 2, 128, 256
    xa = (synth.normal(17, m * k) * 3).astype(np.float32).reshape(m, k)
    qa = np.empty((m, k), np.uint8)
    qs = np.empty((m, k // 128), np.uint8)
    assert R.pr_fp8_quant(_p(xa), m, k, _p(qa), _p(qs)) == 0
    packed, ws = synth.mxfp4_weight(18, n, k)
    o = np.empty((m, n), np.float32)
    assert R.pr_fp4_gemm(_p(qa), _p(qs), _p(packed), _p(ws), m, n, k, _p(o)) == 0
    out.update(fp4_a=qa, fp4_sa=qs, fp4_w=packed, fp4_sw=ws, fp4_out=o)

    # MXFP4 row decode
    rowp, rows = synth.mxfp4_weight(19, 1, 256)
    rows[0, :3] = [0, 126, 200]
    d = np.empty(256, np.float32)
    assert R.pr_mxfp4_decode_row(_p(rowp[0].copy()), _p(rows[0].copy()), 256, _p(d)) == 0
    out.update(mx_packed=rowp[0], mx_scales=rows[0], mx_out=d)

    # SwiGLU (limit 10) and Qwen SiLU-mul
    g = (synth.normal(20, 2 * 64) * 8).astype(np.float32)
    u = (synth.normal(21, 2 * 64) * 8).astype(np.float32)
    sg = np.empty(128, np.float32)
    assert R.pr_swiglu(_p(g), _p(u), 2, 64, 10.0, _p(sg)) == 0
    out.update(swiglu_g=g, swiglu_u=u, swiglu_out=sg)
    gb = synth.bf16_normal(22, (300,), std=3.0)
    ub = synth.bf16_normal(23, (300,))
    so = np.empty(300, np.uint16)
    assert R.pr_silu_mul(_p(gb), _p(ub), 300, _p(so)) == 0
    out.update(silu_g=gb, silu_u=ub, silu_out=so)

    # Routed expert chain (hidden = inter = 128, 3 tokens)
    t, h, it = 3, 128, 128
    xe = synth.bf16_normal(24, (t, h))
    rw = np.array([0.3, 1.0, 0.7], np.float32)
    w1p, w1s = synth.mxfp4_weight(25, it, h)
    w3p, w3s = synth.mxfp4_weight(26, it, h)
    w2p, w2s = synth.mxfp4_weight(27, h, it)
    ye = np.empty((t, h), np.uint16)
    assert R.pr_routed_expert(_p(xe), _p(rw), t, h, it, _p(w1p), _p(w1s), _p(w2p), _p(w2s), _p(w3p), _p(w3s),
                              _p(ye)) == 0
    out.update(re_x=xe, re_w=rw, re_w1p=w1p, re_w1s=w1s, re_w2p=w2p, re_w2s=w2s, re_w3p=w3p, re_w3s=w3s, re_out=ye)

    # Subwave plan (top-6, 256 experts) for 5 tokens
    tokens = 2
    ids, wts = synth.zipf_router(28, tokens, 256, 6)
    expert = ids.astype(np.uint16).ravel()
    token = np.repeat(np.arange(tokens, dtype=np.uint32), 6)
    ordinal = np.tile(np.arange(6, dtype=np.uint8), tokens)
    wt = wts.ravel().astype(np.float32)
    offs = np.empty(257, np.uint32)
    se = np.empty(6 * tokens, np.uint16)
    st = np.empty(6 * tokens, np.uint32)
    so8 = np.empty(6 * tokens, np.uint8)
    sw8 = np.empty(6 * tokens, np.float32)
    assert R.pr_subwave_plan(_p(expert), _p(token), _p(ordinal), _p(wt), tokens, _p(offs), _p(se), _p(st),
                             _p(so8), _p(sw8)) == 0
    out.update(plan_ids=ids, plan_weights=wts, plan_offsets=offs, plan_token=st, plan_weight_sorted=sw8)

    # Ordered accumulate + finalize (hidden 4096 fixed by the reference)
    rows_t = st.astype(np.uint32)
    eo = (synth.normal(29, 6 * tokens * 4096) * 0.5).astype(np.float32).reshape(6 * tokens, 4096)
    eo = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(eo))  # bf16-valued rows
    shared = oracle.bf16_bits_to_f32(synth.bf16_normal(30, (tokens, 4096)))
    res = np.empty((tokens, 4096), np.float32)
    assert R.pr_accumulate(_p(offs), 256, _p(rows_t), _p(eo), tokens, _p(shared), _p(res)) == 0
    out.update(acc_rows=oracle.f32_to_bf16_bits(eo), acc_shared=oracle.f32_to_bf16_bits(shared), acc_out=res)

    # V4 learned router (sqrt-softplus + bias, top-6, x1.5): random scores,
    # a zero-bias token block, and integer scores with exact ties
    rt = 96
    raw = (synth.normal(31, rt * 256) * 3).astype(np.float32).reshape(rt, 256)
    raw[32:64] = np.round(raw[32:64])
    bias = (synth.normal(32, 256) * 0.5).astype(np.float32)
    rid = np.empty((rt, 6), np.uint32)
    rw = np.empty((rt, 6), np.float32)
    assert R.pr_learned_router(_p(raw), rt, _p(bias), _p(rid), _p(rw)) == 0
    out.update(router_raw=raw, router_bias=bias, router_ids=rid, router_weights=rw)

    # Qwen INT4 XINGW4A1 metadata region serialised by the reference for
    # fixed roots and payload digests (the encoded prefix; the rest is zero)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from artifact_files import golden_roots_and_digests  # noqa: E402

    roots, digests = golden_roots_and_digests()
    rb = np.frombuffer(roots, np.uint8).copy()
    db = np.frombuffer(b"".join(digests), np.uint8).copy()
    region = np.zeros(1 << 20, np.uint8)
    enc = np.zeros(1, np.uint32)
    assert R.pr_qwen_int4_metadata(_p(rb), _p(db), _p(region), _p(enc)) == 0
    out["qwen_meta_region"] = region[:int(enc[0])].copy()

    # V4.1 expert FP4 -> FP8 32x32 blocks: random codes with row scales in a
    # narrow band, a band 12 wide (FP8 subnormals and flushes) and one with a
    # maximum of exactly 6
    blocks = 6
    packed = synth.splitmix64(29, blocks * 512).astype(np.uint8).reshape(blocks, 512)
    sc = np.empty((blocks, 32), np.uint8)
    sc[0:2] = (120 + synth.splitmix64(30, 64) % np.uint64(4)).astype(np.uint8).reshape(2, 32)
    sc[2:4] = (100 + synth.splitmix64(31, 64) % np.uint64(13)).astype(np.uint8).reshape(2, 32)
    sc[4] = (synth.splitmix64(32, 32) % np.uint64(7)).astype(np.uint8)
    sc[4, 0] = 6
    sc[5] = 127
    wq = np.empty((blocks, 1024), np.uint8)
    ws = np.empty(blocks, np.uint8)
    for b in range(blocks):
        assert R.pr_v41_fp4_block_to_fp8(_p(packed[b]), _p(sc[b]), _p(wq[b]), _p(ws[b:b + 1])) == 0
    out.update(v41_fp4_packed=packed, v41_fp4_scales=sc, v41_fp8_weight=wq, v41_fp8_scale=ws)

    # V4.1 wo_a block dequantisation (E4M3FN x fp32 scale -> bf16), 32 and 128
    for blk, seed, scale in ((32, 33, 0.0078125 * 1.3), (128, 34, 3.75e-3)):
        src = synth.splitmix64(seed, blk * blk).astype(np.uint8)
        src[(src & 0x7F) == 0x7F] = 0x3C
        dq = np.empty(blk * blk, np.uint16)
        assert R.pr_v41_dequant_block(_p(src), float(np.float32(scale)), blk, _p(dq)) == 0
        out[f"v41_woa{blk}_src"], out[f"v41_woa{blk}_scale"], out[f"v41_woa{blk}_bf16"] = (
            src, np.array([scale], np.float32), dq)

    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
