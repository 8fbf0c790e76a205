"""Pinning of the decode-step oracle (oracle/prism_cpuref_step.c) on the CPU.

Each primitive is checked against the reference's own known-answer tests
where they exist (compute-core/src/lut/evaluator.rs tests), against closed
forms, and against an independent numpy computation; the step itself is
recomposed from the pinned primitives following PrismEngine::step
(src/lut/engine_impl.rs:1076-1405) and must agree bit for bit.
"""
import importlib

import numpy as np
import pytest

import oracle

pe = importlib.import_module("prism-engine_amd")


def f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def val(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


# ---- rms_norm ---------------------------------------------------------------

def test_rms_norm_reference_kat():
    # evaluator.rs:249-257: four ones stay 1.0 within 1e-4
    y = val(oracle.rms_norm(f16([1.0] * 4), 1e-6))
    assert np.all(np.abs(y - 1.0) < 1e-4)


@pytest.mark.parametrize("c", [0.5, -3.0, 0.001, 200.0])
def test_rms_norm_constant_vector(c):
    n = 896
    y = val(oracle.rms_norm(f16([c] * n), 1e-6))
    cf = float(np.float16(c))
    want = np.float16(np.float32(cf) * (np.float32(1.0) / np.sqrt(np.float32(cf * cf) + np.float32(1e-6))))
    assert np.all(y == float(want))


def test_rms_norm_float64_bound_and_scale_invariance():
    rng = np.random.default_rng(1)
    x = f16(rng.standard_normal(896))
    y = val(oracle.rms_norm(x, 1e-6))
    xf = val(x)
    ref = xf / np.sqrt(np.mean(xf * xf) + 1e-6)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)) < 2e-3
    # doubling x (exact in fp16) leaves the output unchanged up to eps
    y2 = val(oracle.rms_norm(f16(2 * xf), 1e-6))
    assert np.max(np.abs(y2 - y)) <= 2 * np.max(np.abs(y)) * 2 ** -10


def test_rms_norm_zero_vector():
    y = oracle.rms_norm(np.zeros(64, np.uint16), 1e-6)
    assert np.all(y == 0)


# ---- vec_add ----------------------------------------------------------------

def test_vec_add_reference_kat():
    # evaluator.rs:258-265: 1 + 2 = 3
    assert np.all(val(oracle.vec_add(f16([1.0] * 4), f16([2.0] * 4))) == 3.0)


def test_vec_add_matches_numpy_float16():
    rng = np.random.default_rng(2)
    a = f16(rng.standard_normal(100000) * 10)
    b = f16(rng.standard_normal(100000) * 10)
    want = (a.view(np.float16) + b.view(np.float16)).view(np.uint16)
    assert np.array_equal(oracle.vec_add(a, b), want)


# ---- rope -------------------------------------------------------------------

def test_rope_pos0_is_identity():
    rng = np.random.default_rng(3)
    x = f16(rng.standard_normal(896))
    assert np.array_equal(oracle.rope(x, 0, 64), x)


@pytest.mark.parametrize("pos", [1, 7, 512, 4095])
def test_rope_pair0_rotates_by_pos_radians(pos):
    rng = np.random.default_rng(4 + pos)
    x = f16(rng.standard_normal(128))
    y = val(oracle.rope(x, pos, 64))
    xf = val(x)
    for head in range(2):
        a, b = xf[head * 64], xf[head * 64 + 32]
        ca, sa = np.cos(pos), np.sin(pos)
        assert abs(y[head * 64] - (a * ca - b * sa)) < 4e-3 * max(1.0, abs(a) + abs(b))
        assert abs(y[head * 64 + 32] - (a * sa + b * ca)) < 4e-3 * max(1.0, abs(a) + abs(b))


def test_rope_angles_and_norm_preservation():
    # angle_j = pos * 10000^(-2j/64) (float64 closed form)
    for j in (0, 1, 5, 31):
        want = 512 * 10000.0 ** (-2 * j / 64)
        assert abs(oracle.rope_angle(512, j, 64) - want) <= 1e-6 * max(1.0, want)
    rng = np.random.default_rng(5)
    x = f16(rng.standard_normal(64))
    y = val(oracle.rope(x, 300, 64))
    xf = val(x)
    for j in range(32):
        n0 = xf[j] ** 2 + xf[j + 32] ** 2
        n1 = y[j] ** 2 + y[j + 32] ** 2
        assert abs(n1 - n0) <= 4e-3 * max(n0, 1e-3)


def test_rope_swapped_pairing_is_detected():
    # plant a mistake in a numpy restatement: pairing (2j, 2j+1) instead of
    # (j, j + hd/2) must disagree with the oracle
    rng = np.random.default_rng(6)
    x = f16(rng.standard_normal(64))
    xf = val(x)
    wrong = xf.copy()
    for j in range(32):
        a, b = xf[2 * j], xf[2 * j + 1]
        ang = 9 * 10000.0 ** (-2 * j / 64)
        wrong[2 * j], wrong[2 * j + 1] = a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)
    assert np.max(np.abs(val(oracle.rope(x, 9, 64)) - wrong)) > 0.1


# ---- INT8 KV ----------------------------------------------------------------

def test_kv_quant_hand_computed_block():
    blk = oracle.kv_quant(f16([1.0, -0.5, 0.25, 0.0]))
    scale = np.frombuffer(blk[:4].tobytes(), dtype="<f4")[0]
    assert scale == np.float32(127.0)
    # 127, -63.5 -> -64 (half away from zero), 31.75 -> 32, 0
    assert blk[4:].view(np.int8).tolist() == [127, -64, 32, 0]


def test_kv_quant_zero_vector_and_empty():
    blk = oracle.kv_quant(np.zeros(8, np.uint16))
    assert np.frombuffer(blk[:4].tobytes(), dtype="<f4")[0] == 1.0
    assert np.all(blk[4:] == 0)
    assert oracle.kv_quant(np.zeros(0, np.uint16)).size == 0


def test_kv_roundtrip_bound():
    rng = np.random.default_rng(7)
    x = f16(rng.standard_normal((20, 128)))
    blocks = np.concatenate([oracle.kv_quant(r) for r in x])
    back = val(oracle.kv_dequant(blocks, 20, 128))
    xf = val(x)
    for t in range(20):
        m = np.max(np.abs(xf[t]))
        # quantization step max/127, half a step error plus fp16 rounding
        assert np.max(np.abs(back[t] - xf[t])) <= m / 254 * 1.01 + 1e-3
        # the largest magnitude maps to +-127
        q = blocks[t * 132 + 4:(t + 1) * 132].view(np.int8)
        assert np.max(np.abs(q.astype(int))) == 127


# ---- attention --------------------------------------------------------------

def test_attention_single_position_returns_v():
    rng = np.random.default_rng(8)
    q = f16(rng.standard_normal(14 * 64))
    k = f16(rng.standard_normal((1, 128)))
    v = f16(rng.standard_normal((1, 128)))
    out = oracle.attention(q, k, v, 14, 2, 64, 1)
    for h in range(14):
        kh = h // 7
        assert np.array_equal(out[h * 64:(h + 1) * 64], v[0, kh * 64:(kh + 1) * 64])


def test_attention_equal_keys_average_values():
    rng = np.random.default_rng(9)
    sl = 9
    q = f16(rng.standard_normal(2 * 64))
    k = np.tile(f16(rng.standard_normal(64)), (sl, 1))
    v = f16(rng.standard_normal((sl, 64)))
    out = val(oracle.attention(q, k, v, 2, 1, 64, sl))
    mean = val(v).mean(axis=0)
    for h in range(2):
        assert np.max(np.abs(out[h * 64:(h + 1) * 64] - mean)) < 2e-3


def test_attention_float64_bound_and_gqa_mapping():
    rng = np.random.default_rng(10)
    nh, nkv, hd, sl = 14, 2, 64, 37
    q = f16(rng.standard_normal(nh * hd))
    k = f16(rng.standard_normal((sl, nkv * hd)))
    v = f16(rng.standard_normal((sl, nkv * hd)))
    out = val(oracle.attention(q, k, v, nh, nkv, hd, sl))
    qf, kf, vf = val(q), val(k), val(v)

    def ref(kh_of):
        o = np.zeros(nh * hd)
        for h in range(nh):
            kh = kh_of(h)
            s = kf[:, kh * hd:(kh + 1) * hd] @ qf[h * hd:(h + 1) * hd] / np.sqrt(hd)
            e = np.exp(s - s.max())
            o[h * hd:(h + 1) * hd] = (e / e.sum()) @ vf[:, kh * hd:(kh + 1) * hd]
        return o

    good = ref(lambda h: h // (nh // nkv))
    assert np.max(np.abs(out - good)) < 4e-3
    # a planted mapping mistake (kv head = h % nkv) is far off
    assert np.max(np.abs(out - ref(lambda h: h % nkv))) > 0.05


# ---- the decode step, recomposed from the pinned pieces ----------------------

TINY = dict(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=256, vocab=300)


def recompose_step(cfg, embed, layers, kv, token, pos):
    """PrismEngine::step (engine_impl.rs:1076-1405) written out in Python
    from the pinned oracle primitives."""
    D, QD, KVD, I, V = cfg.hidden, cfg.q_dim, cfg.kv_dim, cfg.intermediate, cfg.vocab
    h = oracle.lut_embed(token, embed, V, D)
    hr = h.copy()
    for l, (q_p, k_p, v_p, o_p, g_p, u_p, d_p) in enumerate(layers):
        h = oracle.rms_norm(h, cfg.rms_eps)
        q = oracle.gemv(h, q_p, QD, D, 4)[0]
        k = oracle.gemv(h, k_p, KVD, D, 4)[0]
        v = oracle.gemv(h, v_p, KVD, D, 4)[0]
        kv.append(l, k, v)
        q = oracle.rope(q, pos, cfg.head_dim)
        kc, vc = kv.dequant(l)
        h = oracle.attention(q, kc, vc, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, int(kv.len[l]))
        h = oracle.vec_add(oracle.gemv(h, o_p, D, QD, 4)[0], hr)
        hr = h.copy()
        h = oracle.rms_norm(h, cfg.rms_eps)
        gate = oracle.gemv(h, g_p, I, D, 4)[0]
        up = oracle.gemv(h, u_p, I, D, 4)[0]
        act = oracle.swiglu(gate, up)
        h = oracle.vec_add(oracle.gemv(act, d_p, D, I, 4)[0], hr)
        hr = h.copy()
    h = oracle.rms_norm(h, cfg.rms_eps)
    return oracle.gemv(h, embed, V, D, 4)[0]


def tiny_model(seed=11, n_cached=5):
    cfg = pe.Qwen2Config(**TINY)
    embed, layers = pe.synth_weights(cfg, seed)
    emb_p, lay_p = pe.model.payloads(embed, layers)
    kv = oracle.KVState(cfg.n_layers, cfg.kv_dim, 64)
    for l, (k, v) in enumerate(pe.synth_kv(cfg, n_cached, seed)):
        for t in range(n_cached):
            kv.append(l, k[t], v[t])
    return cfg, emb_p, lay_p, kv


@pytest.mark.parametrize("token,pos", [(3, 5), (299, 6), (0, 0), (1000, 2)])
def test_decode_step_matches_recomposition(token, pos):
    cfg, emb_p, lay_p, kv = tiny_model()
    kv2 = kv.copy()
    got = oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv, token, pos, threads=2)
    want = recompose_step(cfg, emb_p, lay_p, kv2, token, pos)
    assert np.array_equal(got, want)
    for l in range(cfg.n_layers):
        assert int(kv.len[l]) == int(kv2.len[l]) == 6
        assert np.array_equal(kv.k[l], kv2.k[l]) and np.array_equal(kv.v[l], kv2.v[l])


def test_decode_step_out_of_range_token_uses_zero_embedding():
    cfg, emb_p, lay_p, kv = tiny_model()
    a = oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv.copy(), 300, 3)
    b = oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv.copy(), 12345, 3)
    assert np.array_equal(a, b)


def test_qwen2_config_from_reference_fixture_values():
    # the values of the reference's tests/fixtures/lut_graph/qwen2_config.json
    d = {"vocab_size": 151936, "hidden_size": 896, "intermediate_size": 4864, "num_hidden_layers": 24,
         "num_attention_heads": 14, "num_key_value_heads": 2, "head_dim": 64, "rms_norm_eps": 1e-6,
         "rope_theta": 1000000, "tie_word_embeddings": True}
    c = pe.Qwen2Config.from_hf(d)
    assert c == pe.Qwen2Config()
    # 7 palettized GEMVs per layer + the tied LM head: 261 574 656 weight bytes
    assert c.weight_bytes() == 261574656
    names = pe.tensor_names(c)
    assert names["embed"] == "model.embed_tokens.weight"
    assert names["layers"][3]["down_proj"] == "model.layers.3.mlp.down_proj.weight"
    assert names["layers"][0]["k_proj"] == "model.layers.0.self_attn.k_proj.weight"
