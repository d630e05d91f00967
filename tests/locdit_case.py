"""Seeded synthetic LocDiT weights and inputs shared by the CPU and GPU tests."""
import numpy as np


def q8(orc, rng, n, k, std=0.02):
    return orc.quantize_rows(rng.normal(0, std, (n, k)).astype(np.float32), orc.QUANT_REF)


def make_locdit(orc, seed, H, L, nh, nkv, hd, F, feat, bias=True):
    """Returns (device config dict, vxm weight dict, oracle LocDiTW, oracle cfg)."""
    rng = np.random.default_rng(seed)
    layers = []
    for _ in range(L):
        layers.append(dict(q_proj=q8(orc, rng, nh * hd, H), k_proj=q8(orc, rng, nkv * hd, H),
                           v_proj=q8(orc, rng, nkv * hd, H), o_proj=q8(orc, rng, H, nh * hd),
                           gate_proj=q8(orc, rng, F, H), up_proj=q8(orc, rng, F, H), down_proj=q8(orc, rng, H, F),
                           input_layernorm=(1 + rng.normal(0, 0.02, H)).astype(np.float32),
                           post_attention_layernorm=(1 + rng.normal(0, 0.02, H)).astype(np.float32)))

    def vec(n, mean=0.0, std=0.02):
        return (mean + rng.normal(0, std, n)).astype(np.float32) if bias else None

    w = dict(layers=layers, in_proj=q8(orc, rng, H, feat, 0.1), in_bias=vec(H),
             cond_proj=q8(orc, rng, H, feat, 0.1), cond_bias=vec(H),
             out_proj=q8(orc, rng, feat, H, 0.05), out_bias=vec(feat),
             norm=(1 + rng.normal(0, 0.02, H)).astype(np.float32),
             t_w1=q8(orc, rng, H, H, 0.03), t_w2=q8(orc, rng, H, H, 0.03),
             dt_w1=q8(orc, rng, H, H, 0.03), dt_w2=q8(orc, rng, H, H, 0.03),
             t_b1=vec(H), t_b2=vec(H), dt_b1=vec(H), dt_b2=vec(H))
    cfg = dict(hidden_size=H, n_layers=L, n_heads=nh, n_kv_heads=nkv, head_dim=hd, intermediate_size=F,
               feat_dim=feat, cond_dim=feat, rms_norm_eps=1e-6, rope_theta=10000)
    lws = [orc.LayerW(wq=d["q_proj"], wk=d["k_proj"], wv=d["v_proj"], wo=d["o_proj"], wg=d["gate_proj"],
                      wu=d["up_proj"], wd=d["down_proj"], g_in=d["input_layernorm"],
                      g_post=d["post_attention_layernorm"]) for d in layers]
    ow = orc.LocDiTW(lws, feat, **{k: v for k, v in w.items() if k != "layers"})
    ocfg = orc.make_cfg(H, nh, nkv, hd, F, eps=1e-6, rope_theta=10000.0,
                        rope_ff=orc.ROPE_SHORT_FACTORS if hd == 128 else None)
    return cfg, w, ow, ocfg


def make_inputs(seed, P, Pc, feat, H):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (P, feat)).astype(np.float32)
    cond = rng.normal(0, 1, (Pc, feat)).astype(np.float32)
    mu = rng.normal(0, 1, (2, H)).astype(np.float32)
    return x, cond, mu
