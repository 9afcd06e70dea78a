"""Stage-by-stage parity of one decoder layer on the GPU (ref
llama_transformer.rs:305-380: RMSNorm, QKV + RoPE + KV append, paged
attention, O + residual, RMSNorm, gate/up + SiLU*up, down + residual).

`run_stages` runs the layer through the public component entry points -- the
same device functions `kcmm_decode_layer_step_on_stream` composes -- and keeps
every intermediate.  `check_stages` compares each stage with the oracle's
stage computed from the GPU's own input to that stage, so an error in one
kernel cannot hide behind the others:

* RMSNorm outputs, q after RoPE, the bf16 K/V rows, the attention output and
  the SwiGLU activation: max |got - ref| <= tol * max |ref| (tol 1e-2; the
  attention on an fp8 pool 3e-2, its tolerance in the north star);
* fp8 K/V rows: within one e4m3 step (2^-3 relative, 2^-9 * scale near 0) of
  the oracle's bf16 row, plus one bf16 step for the rounding of that row;
* O + residual and down + residual store bf16(x + bf16(p)) for a projection
  p: the projection's part must be within tol * max |p_ref| and the sum may
  differ by the one bf16 rounding of the sum (2^-8 * |ref|).

Measured errors are returned so the caller can print and bound them.
"""
import numpy as np

import oracle as O
from lattice_amd.bindings import KV_FP8, memcpy_dtoh

BF16_STEP = 2.0 ** -8     # spacing of bf16 values relative to the value


def _dev(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def _bits(t):
    import torch
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _f64(bits):
    return O.decode(O.BF16, bits).astype(np.float64)


def rel_err(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def residual_err(got, ref, x):
    """Error of bf16(x + bf16(p)) beyond the one rounding of the sum, relative
    to max |p_ref| (p_ref = ref - x)."""
    slack = BF16_STEP * np.abs(ref)
    over = np.maximum(np.abs(got - ref) - slack, 0.0)
    return float(over.max() / max(np.abs(ref - x).max(), 1e-30))


def attn_scale(d):
    return float(np.float32(1.0) / np.sqrt(np.float32(d)))


def run_stages(lib, case, wdev, hid_bits, invd, hq, h, inter, eps, stream):
    """Runs the layer for layer 0 of `case` one component at a time; returns
    the bf16 bits of every stage plus the K/V regions before / after the
    append."""
    import torch
    g = case.geometry
    pool, dv = case.pool, case.dev
    d = case.head_dim
    B = hid_bits.shape[0]
    nbytes = g["mapped_bytes"]
    e = lambda *shape: torch.full(shape, float("nan"), dtype=torch.bfloat16, device="cuda")
    x = _dev(torch, hid_bits)
    n1, q, att, n2, act = e(B, h), e(B, hq * d), e(B, hq * d), e(B, h), e(B, inter)
    kv0 = (memcpy_dtoh(pool.va_k(0), nbytes), memcpy_dtoh(pool.va_v(0), nbytes))
    lib.rmsnorm_bf16(x.data_ptr(), wdev["attn_norm"].data_ptr(), n1.data_ptr(), B, h, eps, stream)
    common = dict(layer_idx=0, q_out_ptr=q.data_ptr(), block_tables_ptr=dv["bt"].data_ptr(),
                  seq_lens_ptr=dv["sl"].data_ptr(), block_offsets_f16_ptr=dv["offs"].data_ptr(),
                  inv_freq_ptr=invd.data_ptr(), batch=B, num_q_heads=hq,
                  max_blocks_per_seq=case.mbps, stream_ptr=stream)
    if d % 16 == 0:
        pool.qkv_rope_append(x_ptr=n1.data_ptr(), w_qkv_ptr=wdev["qkv"].data_ptr(),
                             hidden_size=h, **common)
    else:   # the layer step's unfused path: projection, then RoPE + append
        qkv = e(B, (hq + 2 * case.kv_heads) * d)
        lib.gemm_bf16(n1.data_ptr(), wdev["qkv"].data_ptr(), qkv.data_ptr(), B, qkv.shape[1], h,
                      stream)
        pool.rope_append(qkv_ptr=qkv.data_ptr(), **common)
    torch.cuda.synchronize()
    kv1 = (memcpy_dtoh(pool.va_k(0), nbytes), memcpy_dtoh(pool.va_v(0), nbytes))
    pool.paged_attn_decode(layer_idx=0, query_ptr=q.data_ptr(), out_ptr=att.data_ptr(),
                           block_tables_ptr=dv["bt"].data_ptr(), seq_lens_ptr=dv["sl"].data_ptr(),
                           block_offsets_f16_ptr=dv["offs"].data_ptr(), batch=B, num_q_heads=hq,
                           kv_heads=case.kv_heads, head_dim=d, block_size=case.block_size,
                           max_blocks_per_seq=case.mbps, scale=attn_scale(d), stream_ptr=stream)
    h1 = x.clone()
    lib.gemm_bf16_add_rmsnorm(att.data_ptr(), wdev["o"].data_ptr(), h1.data_ptr(),
                              wdev["mlp_norm"].data_ptr(), n2.data_ptr(), B, h, hq * d, eps,
                              stream)
    lib.gemm_bf16_swiglu(n2.data_ptr(), wdev["gate_up"].data_ptr(), act.data_ptr(), B, inter, h,
                         stream)
    out = h1.clone()
    lib.gemm_bf16_add(act.data_ptr(), wdev["down"].data_ptr(), out.data_ptr(), out.data_ptr(), B,
                      h, inter, stream)
    torch.cuda.synchronize()
    return {"x": hid_bits, "n1": _bits(n1), "q": _bits(q), "att": _bits(att), "h1": _bits(h1),
            "n2": _bits(n2), "act": _bits(act), "out": _bits(out), "kv0": kv0, "kv1": kv1}


def check_stages(st, case, w, inv, hq, inter, eps, dtype, tol=1e-2):
    """Compares every stage of `run_stages` with the oracle; returns the
    measured errors (asserting each one)."""
    g = case.geometry
    hkv, d, bs = case.kv_heads, case.head_dim, case.block_size
    rb, db = g["row_bytes"], g["data_bytes"]
    fp8 = dtype == KV_FP8
    f = lambda name: O.layer_weight_f64(w, name)
    rnd = O.bf16_round
    B = st["x"].shape[0]
    errs = {}
    x = _f64(st["x"])
    # RMSNorm 1
    errs["norm1"] = rel_err(_f64(st["n1"]), O.rmsnorm_f64(x, f("attn_norm"), eps, True))
    # QKV + RoPE (q rotated; k rotated and v into the new token's page row)
    n1 = _f64(st["n1"])
    qkv = rnd(n1 @ f("qkv").T)
    pos = np.asarray(case.seq_lens, np.int64) - 1
    pe = np.maximum(pos, 0)[:, None].astype(np.float64)
    q_r = rnd(O.rope_f64(qkv[:, :hq * d].reshape(B, hq, d), pe, inv))
    k_r = rnd(O.rope_f64(qkv[:, hq * d:(hq + hkv) * d].reshape(B, hkv, d), pe, inv))
    v_n = qkv[:, (hq + hkv) * d:].reshape(B, hkv, d)
    live = pos >= 0
    errs["q_rope"] = rel_err(_f64(st["q"]).reshape(B, hq, d)[live], q_r[live])
    kv_err, fp8_over = 0.0, 0.0
    changed = [np.zeros(st["kv0"][0].size, bool) for _ in range(2)]
    for b in np.nonzero(live)[0]:
        p = int(pos[b])
        page = int(case.offsets_f16[case.block_tables[b, p // bs]]) * 2
        at = page + (p % bs) * rb
        for which, ref in ((0, k_r[b]), (1, v_n[b])):
            reg = st["kv1"][which]
            if fp8:
                got = O.fp8_page_rows(reg, page, [p % bs], hkv, d, rb, db)[0]
                sc = reg[page + db:page + db + 4 * hkv].view(np.float32).astype(np.float64)
                bound = (2.0 ** -3 + BF16_STEP) * np.abs(ref) + 2.0 ** -9 * sc[:, None]
                fp8_over = max(fp8_over, float((np.abs(got - ref) / bound).max()))
                changed[which][at:at + hkv * d] = True
                changed[which][page + db:page + db + 4 * hkv] = True
                # the page's other rows are re-encoded when its scale grows
                changed[which][page:page + db] = True
            else:
                got = _f64(reg[at:at + hkv * d * 2].view(np.uint16)).reshape(hkv, d)
                kv_err = max(kv_err, rel_err(got, ref))
                changed[which][at:at + hkv * d * 2] = True
    for which in range(2):
        same = st["kv0"][which] == st["kv1"][which]
        assert same[~changed[which]].all(), "the append changed bytes outside the new rows"
    if fp8:
        errs["kv_rows_fp8_bound_frac"] = fp8_over
    else:
        errs["kv_rows"] = kv_err
    # attention over the GPU's pages (fp8: dequantized) with the GPU's q
    att_ref = O.attn_decode_f64(dtype, st["q"], st["kv1"][0], st["kv1"][1], case.block_tables,
                                case.seq_lens, case.offsets_f16, hq, hkv, d, bs, rb, db,
                                attn_scale(d))
    errs["attn"] = rel_err(_f64(st["att"]), att_ref.reshape(B, hq * d))
    # O + residual, RMSNorm 2
    att = _f64(st["att"])
    h1_ref = rnd(x + rnd(att @ f("o").T))
    errs["o_residual"] = residual_err(_f64(st["h1"]), h1_ref, x)
    h1 = _f64(st["h1"])
    errs["norm2"] = rel_err(_f64(st["n2"]), O.rmsnorm_f64(h1, f("mlp_norm"), eps, True))
    # gate/up + SwiGLU
    gu = rnd(_f64(st["n2"]) @ f("gate_up").T)
    gg = gu[:, :inter]
    with np.errstate(over="ignore"):
        act_ref = rnd(rnd(gg / (1.0 + np.exp(-gg))) * gu[:, inter:])
    errs["swiglu"] = rel_err(_f64(st["act"]), act_ref)
    # down + residual
    out_ref = rnd(h1 + rnd(_f64(st["act"]) @ f("down").T))
    errs["down_residual"] = residual_err(_f64(st["out"]), out_ref, h1)
    limits = {k: tol for k in errs}
    limits["attn"] = 3e-2 if fp8 else tol
    limits["kv_rows_fp8_bound_frac"] = 1.0
    for k, v in errs.items():
        assert np.isfinite(v) and v <= limits[k], (k, v, limits[k])
    return errs
