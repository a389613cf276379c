"""Oracle vs the committed brute-force golden vectors (CPU only)."""

import numpy as np

import oracle

TOL = dict(rtol=1e-2, atol=2e-2)  # bf16 outputs: one-ulp flips between fp32 and fp64 pipelines


def test_gemv(golden):
    np.testing.assert_allclose(oracle.gemv(golden["gemv_x"], golden["gemv_W"]), golden["gemv_y"], **TOL)


def test_rmsnorm(golden):
    np.testing.assert_allclose(oracle.rmsnorm_f32(golden["rms32_X"]), golden["rms32_out"], rtol=1e-6)
    np.testing.assert_allclose(oracle.rmsnorm_bf16(golden["rmsbf_X"], golden["rmsbf_w"]), golden["rmsbf_out"], **TOL)


def test_softmax_reduce(golden):
    np.testing.assert_allclose(oracle.softmax(golden["softmax_X"]), golden["softmax_out"], rtol=1e-6)
    np.testing.assert_array_equal(oracle.reduce_sum(golden["reduce_A"]), golden["reduce_out"])


def test_attn(golden):
    y = oracle.attn_decode(golden["attn_Q"], golden["attn_K"], golden["attn_V"], golden["attn_lens"])
    np.testing.assert_allclose(y, golden["attn_out"], **TOL)


def test_qk_norm_rope(golden):
    g = golden
    q, k, Kc, Vc = oracle.qk_norm_rope(g["rope_q"], g["rope_k"], g["rope_v"], g["rope_qw"], g["rope_kw"],
                                       g["rope_cos"], g["rope_sin"], g["rope_Kc"], g["rope_Vc"], g["rope_pos"])
    np.testing.assert_allclose(q, g["rope_qout"], **TOL)
    np.testing.assert_allclose(k, g["rope_kout"], **TOL)
    for b, p in enumerate(g["rope_pos"]):
        np.testing.assert_array_equal(Vc[b, :, p], g["rope_v"][b])


def test_o_proj_ffn(golden):
    g = golden
    y = oracle.o_proj_ffn(g["ffn_attn"], g["ffn_res"], g["ffn_Wo"], g["ffn_w"], g["ffn_Wg"], g["ffn_Wu"], g["ffn_Wd"])
    np.testing.assert_allclose(y, g["ffn_out"], **TOL)


def test_qwen3_layer(golden):
    g = golden
    out, Kc, Vc = oracle.qwen3_layer(
        g["layer_hidden"], g["layer_Kc"], g["layer_Vc"], g["layer_Wqkv"], g["layer_Wo"], g["layer_Wgu"],
        g["layer_Wd"], 4, 2, 8, kv_lens=g["layer_lens"], in_norm_w=g["layer_inw"], q_norm_w=g["layer_qw"],
        k_norm_w=g["layer_kw"], post_norm_w=g["layer_pw"], cos=g["layer_cos"], sin=g["layer_sin"])
    np.testing.assert_allclose(out, g["layer_out"], **TOL)
    np.testing.assert_allclose(Kc, g["layer_Kc_out"], **TOL)
    np.testing.assert_allclose(Vc, g["layer_Vc_out"], **TOL)
