"""Pins the decode-step glue and layer-step oracle (oracle.rmsnorm_f64,
rope_f64, silu_mul_f64, default_inv_freq, decode_layer_step_f64) against the
Hugging Face Llama modules (transformers, run on the CPU in float64), plus the
invariants RoPE must keep.  The reference's own rope.cu pairs and theta are not
HF's (ref src/model/llama_transformer.rs:324-330); HF semantics are the
target."""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
ml = pytest.importorskip("transformers.models.llama.modeling_llama")
from transformers import LlamaConfig  # noqa: E402
from transformers.cache_utils import DynamicCache  # noqa: E402


def cfg(h=256, inter=512, hq=4, hkv=2, d=64, theta=500000.0, eps=1e-5, rope_parameters=None):
    c = LlamaConfig(hidden_size=h, intermediate_size=inter, num_attention_heads=hq,
                    num_key_value_heads=hkv, head_dim=d, rms_norm_eps=eps, rope_theta=theta,
                    max_position_embeddings=8192)
    if rope_parameters is not None:
        c.rope_parameters = rope_parameters
    c._attn_implementation = "eager"
    return c


def bf16_vals(rng, shape, std=1.0):
    return O.decode(O.BF16, O.encode(O.BF16, rng.standard_normal(shape) * std)).astype(np.float64)


def test_rmsnorm_matches_hf():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 256))
    w = 1.0 + 0.1 * rng.standard_normal(256)
    m = ml.LlamaRMSNorm(256, eps=1e-5).double()
    m.weight.data = torch.from_numpy(w)
    with torch.no_grad():
        ref = m(torch.from_numpy(x)).numpy()
    # (HF normalises in float32 whatever the input type)
    assert np.allclose(O.rmsnorm_f64(x, w, 1e-5, round_bf16=False), ref, rtol=1e-6, atol=1e-6)
    # bf16 model: the normalised row is rounded before the weight multiply
    xb, wb = bf16_vals(rng, (5, 256)), bf16_vals(rng, 256) + 1.0
    wb = O.bf16_round(wb)
    mb = ml.LlamaRMSNorm(256, eps=1e-5).to(torch.bfloat16)
    mb.weight.data = torch.from_numpy(wb).to(torch.bfloat16)
    with torch.no_grad():
        refb = mb(torch.from_numpy(xb).to(torch.bfloat16)).float().numpy()
    got = O.rmsnorm_f64(xb, wb, 1e-5)
    ulp = np.abs(refb) * 2.0 ** -7
    assert np.all(np.abs(got - refb) <= ulp + 1e-30)
    assert np.mean(got == refb) > 0.99


def test_default_inv_freq_matches_hf():
    rot = ml.LlamaRotaryEmbedding(cfg(d=128, theta=500000.0))
    ref = rot.inv_freq.double().numpy()
    assert np.allclose(O.default_inv_freq(500000.0, 128), ref, rtol=1e-6)


@pytest.mark.parametrize("rope", [None, {"rope_type": "llama3", "rope_theta": 500000.0,
                                         "factor": 8.0, "low_freq_factor": 1.0,
                                         "high_freq_factor": 4.0,
                                         "original_max_position_embeddings": 8192}])
def test_rope_matches_hf(rope):
    """HF apply_rotary_pos_emb with its own cos/sin (default and llama3
    frequency tables) equals rope_f64 given the same inv_freq table."""
    c = cfg(d=64, rope_parameters=rope)
    rot = ml.LlamaRotaryEmbedding(c)
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 4, 3, 64))
    k = rng.standard_normal((1, 2, 3, 64))
    pos = np.array([[0, 7, 45]])
    with torch.no_grad():
        cos, sin = rot(torch.zeros(1, 3, 64, dtype=torch.float64), torch.from_numpy(pos))
        rq, rk = ml.apply_rotary_pos_emb(torch.from_numpy(q), torch.from_numpy(k), cos.double(),
                                         sin.double())
    inv = rot.inv_freq.double().numpy()
    p = pos.reshape(1, 1, 3).astype(np.float64)
    assert np.allclose(O.rope_f64(q, p, inv), rq.numpy(), rtol=1e-5, atol=1e-5)
    assert np.allclose(O.rope_f64(k, p, inv), rk.numpy(), rtol=1e-5, atol=1e-5)


def test_rope_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 128))
    inv = O.default_inv_freq(10000.0, 128)
    assert np.allclose(O.rope_f64(x, np.zeros(6), inv), x)               # position 0
    y = O.rope_f64(x, np.full(6, 37.0), inv)
    pair = lambda a: a[:, :64] ** 2 + a[:, 64:] ** 2                      # (i, i + D/2) norms
    assert np.allclose(pair(y), pair(x))
    z = O.rope_f64(O.rope_f64(x, np.full(6, 11.0), inv), np.full(6, 26.0), inv)
    assert np.allclose(z, y)                                              # rotations add
    # a planted pairing mistake (i, i + 1) breaks the pair-norm invariant
    bad = x.copy()
    bad[:, 0::2], bad[:, 1::2] = y[:, :64], y[:, 64:]
    assert not np.allclose(pair(bad), pair(x))


def test_silu_mul_matches_torch():
    rng = np.random.default_rng(4)
    g, u = rng.standard_normal((3, 40)) * 4, rng.standard_normal((3, 40))
    ref = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    assert np.allclose(O.silu_mul_f64(g, u), ref, rtol=1e-12, atol=1e-12)


def _layer_case(rng, h, inter, hq, hkv, d, bs, lens):
    """Random bf16 weights / hidden / past K,V in a synthetic page layout
    (page i at byte offset i * page_bytes, pages handed out in order)."""
    row_bytes = hkv * d * 2
    page_bytes = bs * row_bytes
    mbps = max((L + bs - 1) // bs for L in lens)
    n_pages = sum((L + bs - 1) // bs for L in lens)
    bt = np.zeros((len(lens), mbps), dtype=np.int32)
    nxt = 0
    for b, L in enumerate(lens):
        for j in range((L + bs - 1) // bs):
            bt[b, j] = nxt
            nxt += 1
    offs = (np.arange(n_pages, dtype=np.uint64) * page_bytes) // 2
    kreg = O.encode(O.BF16, rng.standard_normal(n_pages * page_bytes // 2)).view(np.uint8).copy()
    vreg = O.encode(O.BF16, rng.standard_normal(n_pages * page_bytes // 2)).view(np.uint8).copy()
    enc = lambda shape, std: O.encode(O.BF16, rng.standard_normal(shape) * std)
    w = {"attn_norm": O.encode(O.BF16, 1.0 + 0.1 * rng.standard_normal(h)),
         "qkv": enc(((hq + 2 * hkv) * d, h), 0.05), "o": enc((h, hq * d), 0.05),
         "mlp_norm": O.encode(O.BF16, 1.0 + 0.1 * rng.standard_normal(h)),
         "gate_up": enc((2 * inter, h), 0.05), "down": enc((h, inter), 0.05)}
    hidden = O.encode(O.BF16, rng.standard_normal((len(lens), h)))
    return dict(w=w, hidden=hidden, kreg=kreg, vreg=vreg, bt=bt, offs=offs,
                sl=np.array(lens, dtype=np.int32), row_bytes=row_bytes)


def test_layer_step_matches_hf_decoder_layer():
    """The layer-step oracle without bf16 rounding equals transformers'
    LlamaDecoderLayer (float64, eager attention over a cache holding the
    sequence's earlier K/V rows from the pages)."""
    h, inter, hq, hkv, d, bs, eps = 256, 512, 4, 2, 64, 16, 1e-5
    lens = [5, 17, 33]
    rng = np.random.default_rng(5)
    cs = _layer_case(rng, h, inter, hq, hkv, d, bs, lens)
    c = cfg(h, inter, hq, hkv, d, eps=eps)
    rot = ml.LlamaRotaryEmbedding(c)
    inv = rot.inv_freq.double().numpy()
    kreg0, vreg0 = cs["kreg"].copy(), cs["vreg"].copy()
    got = O.decode_layer_step_f64(cs["hidden"], cs["w"], cs["kreg"], cs["vreg"], cs["bt"],
                                  cs["sl"], cs["offs"], inv, hq, hkv, d, inter, bs,
                                  cs["row_bytes"], eps, round_bf16=False)
    layer = ml.LlamaDecoderLayer(c, layer_idx=0).double()
    W = {k: torch.from_numpy(O.decode(O.BF16, v).astype(np.float64)) for k, v in cs["w"].items()}
    with torch.no_grad():
        layer.input_layernorm.weight.copy_(W["attn_norm"])
        layer.self_attn.q_proj.weight.copy_(W["qkv"][:hq * d])
        layer.self_attn.k_proj.weight.copy_(W["qkv"][hq * d:(hq + hkv) * d])
        layer.self_attn.v_proj.weight.copy_(W["qkv"][(hq + hkv) * d:])
        layer.self_attn.o_proj.weight.copy_(W["o"])
        layer.post_attention_layernorm.weight.copy_(W["mlp_norm"])
        layer.mlp.gate_proj.weight.copy_(W["gate_up"][:inter])
        layer.mlp.up_proj.weight.copy_(W["gate_up"][inter:])
        layer.mlp.down_proj.weight.copy_(W["down"])
    x = O.decode(O.BF16, cs["hidden"]).astype(np.float64)
    for b, L in enumerate(lens):
        pos = L - 1
        past_k = np.zeros((1, hkv, pos, d))
        past_v = np.zeros((1, hkv, pos, d))
        for t in range(pos):
            base = int(cs["offs"][cs["bt"][b, t // bs]]) * 2 + (t % bs) * cs["row_bytes"]
            seg = slice(base, base + hkv * d * 2)
            past_k[0, :, t] = O.decode(O.BF16, kreg0[seg].view(np.uint16)).reshape(hkv, d)
            past_v[0, :, t] = O.decode(O.BF16, vreg0[seg].view(np.uint16)).reshape(hkv, d)
        cache = DynamicCache()
        if pos > 0:
            cache.update(torch.from_numpy(past_k), torch.from_numpy(past_v), 0)
        hs = torch.from_numpy(x[b][None, None, :])
        pid = torch.tensor([[pos]])
        with torch.no_grad():
            cos, sin = rot(hs, pid)
            ref = layer(hs, attention_mask=None, position_ids=pid, past_key_values=cache,
                        use_cache=True, position_embeddings=(cos.double(), sin.double()))
        ref = ref.numpy()[0, 0]
        assert np.allclose(got[b], ref, rtol=1e-5, atol=1e-5), (b, np.abs(got[b] - ref).max())


def test_layer_step_rounding_is_small_and_writes_pages():
    """The bf16 layer stays within bf16 noise of the fp64 one, and only the
    new token's rows of the pages change."""
    h, inter, hq, hkv, d, bs, eps = 256, 512, 4, 2, 64, 16, 1e-5
    lens = [1, 16, 20]
    rng = np.random.default_rng(6)
    cs = _layer_case(rng, h, inter, hq, hkv, d, bs, lens)
    inv = O.default_inv_freq(500000.0, d)
    k1, v1, k2, v2 = (cs["kreg"].copy(), cs["vreg"].copy(), cs["kreg"].copy(),
                      cs["vreg"].copy())
    args = (cs["bt"], cs["sl"], cs["offs"], inv, hq, hkv, d, inter, bs, cs["row_bytes"], eps)
    a = O.decode_layer_step_f64(cs["hidden"], cs["w"], k1, v1, *args)
    b = O.decode_layer_step_f64(cs["hidden"], cs["w"], k2, v2, *args, round_bf16=False)
    assert np.abs(a - b).max() <= 2e-2 * np.abs(b).max()
    changed = np.flatnonzero((k1 != cs["kreg"]) | (v1 != cs["vreg"]))
    rows = set()
    for i in changed:
        rows.add(int(i) // cs["row_bytes"])
    want = set()
    for bb, L in enumerate(lens):
        p = L - 1
        want.add((int(cs["offs"][cs["bt"][bb, p // bs]]) * 2 + (p % bs) * cs["row_bytes"])
                 // cs["row_bytes"])
    assert rows <= want


def test_layer_step_fp8_weights_equal_exact_bf16_weights():
    """fp8-weight projections given as (e4m3 codes, row scales): with
    power-of-two row scales every weight code * scale is a bf16 value, so the
    layer must equal the bf16 layer on those values bit for bit; a dropped or
    misapplied row scale (scales differ per row) breaks the equality."""
    h, inter, hq, hkv, d, bs, eps = 256, 512, 4, 2, 64, 16, 1e-5
    lens = [1, 16, 20]
    rng = np.random.default_rng(8)
    cs = _layer_case(rng, h, inter, hq, hkv, d, bs, lens)
    inv = O.default_inv_freq(500000.0, d)
    w8, wexact = dict(cs["w"]), dict(cs["w"])
    for name in ("qkv", "o", "gate_up", "down"):
        n, k = cs["w"][name].shape
        codes = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
        codes[(codes & 0x7F) == 0x7F] = 0x38          # no NaN codes
        scale = (2.0 ** rng.integers(-9, -5, size=n)).astype(np.float32)
        w8[name] = (codes, scale)
        deq = O.decode(O.FP8, codes).astype(np.float64) * scale[:, None]
        wexact[name] = O.encode(O.BF16, deq)
        assert np.array_equal(O.decode(O.BF16, wexact[name]).astype(np.float64), deq)
    args = (cs["bt"], cs["sl"], cs["offs"], inv, hq, hkv, d, inter, bs, cs["row_bytes"], eps)
    k1, v1, k2, v2 = (cs["kreg"].copy(), cs["vreg"].copy(), cs["kreg"].copy(),
                      cs["vreg"].copy())
    a = O.decode_layer_step_f64(cs["hidden"], w8, k1, v1, *args)
    b = O.decode_layer_step_f64(cs["hidden"], wexact, k2, v2, *args)
    assert np.array_equal(a, b) and np.array_equal(k1, k2) and np.array_equal(v1, v2)
    # the scale matters: the same codes at scale 1 give another layer
    w1 = {k: ((v[0], np.ones_like(v[1])) if isinstance(v, tuple) else v) for k, v in w8.items()}
    c = O.decode_layer_step_f64(cs["hidden"], w1, cs["kreg"].copy(), cs["vreg"].copy(), *args)
    assert not np.allclose(a, c)
