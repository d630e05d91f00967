"""Benchmark of the Q8_0 matmul hot path on one MI355X.

Workload (the "step"): one decode token through a 28-layer MiniCPM4-style
stack (hidden 2048, 16 q / 2 kv heads of 128, SwiGLU 6144, Q8_0 weights
~ N(0, 0.02) from seed 1), batch 1, f16 KV cache growing from context 256 to
320 over 64 tokens, weights rotated through 3 device copies (4.2 GB, far
beyond the 256 MB Infinity Cache).  `value` is the algorithmic weight + KV
bytes of a step over its time (GB/s); the line also carries us per step, the
isolated Q8_0 GEMV (6144x2048 and 2048x6144 over 64 rotated copies), one
decoder layer step at context 512, the 512-token prefill, the CFM solve, the
per-token LM update (LocEnc + TSLM + FSQ + RALM), the roofline of the
dominant kernel and the host-CPU baseline (the oracle's SIMD restatement of
ggml's CPU path).

--gpus above 1 is refused: this build runs on one GPU.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "voxcpm-cpp_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA
H, NH, NKV, HD, F, L = 2048, 16, 2, 128, 6144, 28


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_persistent_28L_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE scaled against a copy kernel), or None when the summary is absent."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic bytes per launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def log(msg):
    print(f"# {msg}", file=sys.stderr, flush=True)


def q8_bytes(n, k):
    return n * k // 32 * 34


def gemv_bytes(n, k):
    # weights + quantized activation (K int8 + K/32 fp16 scales) + fp32 output
    return q8_bytes(n, k) + k + k // 32 * 2 + 4 * n


def layer_weight_bytes():
    qd, kvd = NH * HD, NKV * HD
    return (q8_bytes(qd, H) + 2 * q8_bytes(kvd, H) + q8_bytes(H, qd) + 2 * q8_bytes(F, H) + q8_bytes(H, F))


def step_bytes(ctx_len, n_layers=L):
    """Algorithmic HBM bytes of one decode token: Q8_0 weights, gains, KV read + append."""
    kv_read = 2 * NKV * HD * 2 * (ctx_len + 1)
    return n_layers * (layer_weight_bytes() + 2 * H * 4 + kv_read)


def make_layers(vxm, seed, n_layers, hidden=H, nh=NH, nkv=NKV, hd=HD, ffn=F):
    """Seeded synthetic Q8_0 layers (GGUF rows) and gains."""
    H, qd, kvd, F = hidden, nh * hd, nkv * hd, ffn
    shapes = [("q_proj", qd, H), ("k_proj", kvd, H), ("v_proj", kvd, H), ("o_proj", H, qd),
              ("gate_proj", F, H), ("up_proj", F, H), ("down_proj", H, F)]
    per_layer = sum(n * k for _, n, k in shapes) + 2 * H
    layers = []
    for l in range(n_layers):
        off = l * per_layer
        d = {}
        for name, n, k in shapes:
            w = vxm.host_randn(seed, n * k, 0.0, 0.02, offset=off).reshape(n, k)
            d[name] = vxm.host_quantize_q8_0(w)
            off += n * k
        d["input_layernorm"] = vxm.host_randn(seed, H, 1.0, 0.02, offset=off)
        d["post_attention_layernorm"] = vxm.host_randn(seed, H, 1.0, 0.02, offset=off + H)
        layers.append(d)
    return layers


def kv_prefill(vxm, kv, n_layers, ctx_len, seed):
    """Cache rows [0, ctx_len) of every layer from N(0,1), BF16-representable f16."""
    import numpy as np

    import torch

    for l in range(n_layers):
        ks = []
        for j in range(2):
            v = vxm.host_randn(seed + 100 + l, NKV * kv.cap * HD, 0.0, 1.0, offset=j * NKV * kv.cap * HD)
            v = v.reshape(NKV, kv.cap, HD)
            v[:, ctx_len:] = 0.0
            bf = torch.from_numpy(v).to(torch.bfloat16).to(torch.float16).numpy().view(np.uint16)
            ks.append(bf)
        kv.upload(l, ks[0], ks[1])
    kv.set_used(ctx_len)


class Timer:
    """HIP events on the library's stream."""

    def __init__(self, torch, ctx):
        self.torch, self.st = torch, ctx.torch_stream()
        self.e0 = torch.cuda.Event(enable_timing=True)
        self.e1 = torch.cuda.Event(enable_timing=True)

    def start(self):
        self.e0.record(self.st)

    def stop_ms(self):
        self.e1.record(self.st)
        self.e1.synchronize()
        return self.e0.elapsed_time(self.e1)


def bench_gemv(ctx, torch, vxm, N, K, copies, reps):
    import numpy as np

    w32 = vxm.host_randn(0, N * K, 0.0, 0.02).reshape(N, K)
    x = vxm.host_randn(0, K, 0.0, 1.0, offset=N * K).reshape(1, K)
    wq = vxm.host_quantize_q8_0(w32)
    ws = [ctx.upload_q8_0(wq, N, K) for _ in range(copies)]
    xq, xs = ctx.quantize_q8_0(torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0"), vxm.QUANT_X86)
    y = torch.empty((1, N), dtype=torch.float32, device="cuda:0")
    L_ = vxm.lib()
    args = [(w.h, vxm._ptr(xq), vxm._ptr(xs), vxm._ptr(y)) for w in ws]
    for a in args:
        L_.vxm_mul_mat_q8_0_q8_0(ctx.h, a[0], a[1], a[2], 1, a[3])
    ctx.sync()
    t = Timer(torch, ctx)
    t.start()
    for _ in range(reps):
        for a in args:
            L_.vxm_mul_mat_q8_0_q8_0(ctx.h, a[0], a[1], a[2], 1, a[3])
    us = t.stop_ms() * 1000.0 / (reps * copies)
    for w in ws:
        w.free()
    return us


def bench_gemv_multi(ctx, torch, vxm, N, K, copies, reps):
    """`copies` rotated copies of one GEMV in ONE launch (vxm_mul_mat_q8_0_q8_0_multi), launches back to
    back: us per launch (all copies)."""
    import ctypes as C

    import numpy as np

    w32 = vxm.host_randn(0, N * K, 0.0, 0.02).reshape(N, K)
    x = vxm.host_randn(0, K, 0.0, 1.0, offset=N * K).reshape(1, K)
    wq = vxm.host_quantize_q8_0(w32)
    ws = [ctx.upload_q8_0(wq, N, K) for _ in range(copies)]
    xq, xs = ctx.quantize_q8_0(torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0"), vxm.QUANT_X86)
    ys = [torch.empty((1, N), dtype=torch.float32, device="cuda:0") for _ in range(copies)]
    arr = C.c_void_p * copies
    a_w = arr(*[w.h.value for w in ws])
    a_q = arr(*[xq.data_ptr()] * copies)
    a_s = arr(*[xs.data_ptr()] * copies)
    a_y = arr(*[y.data_ptr() for y in ys])
    L_ = vxm.lib()
    ctx.check(L_.vxm_mul_mat_q8_0_q8_0_multi(ctx.h, copies, a_w, a_q, a_s, 1, a_y))
    ctx.sync()
    ref = ctx.mul_mat_q8(ws[0], xq, xs)
    same = all(bool(torch.equal(y, ref)) for y in ys)
    t = Timer(torch, ctx)
    t.start()
    for _ in range(reps):
        L_.vxm_mul_mat_q8_0_q8_0_multi(ctx.h, copies, a_w, a_q, a_s, 1, a_y)
    us = t.stop_ms() * 1000.0 / reps
    for w in ws:
        w.free()
    return us, same


def bench_read_floor(ctx, torch, vxm, nbytes, copies, reps, per_launch):
    """vxm_stream_read over `copies` buffers of nbytes: `per_launch` buffers per launch, launches back to
    back over the rotation.  Returns us per buffer read."""
    import ctypes as C

    n16 = (nbytes + 15) // 16
    bufs = [torch.ones(n16 * 4, dtype=torch.int32, device="cuda:0") for _ in range(copies)]
    groups = [bufs[i:i + per_launch] for i in range(0, copies, per_launch)]
    args = []
    for g in groups:
        args.append((len(g), (C.c_void_p * len(g))(*[b.data_ptr() for b in g]),
                     (C.c_int64 * len(g))(*[n16 * 16] * len(g))))
    L_ = vxm.lib()
    words = max(L_.vxm_stream_read_sink_words(n, b) for n, _, b in args)
    sink = torch.zeros(words, dtype=torch.int32, device="cuda:0")
    for n, p, b in args:
        ctx.check(L_.vxm_stream_read(ctx.h, n, p, b, C.c_void_p(sink.data_ptr())))
    ctx.sync()
    t = Timer(torch, ctx)
    t.start()
    for _ in range(reps):
        for n, p, b in args:
            L_.vxm_stream_read(ctx.h, n, p, b, C.c_void_p(sink.data_ptr()))
    us = t.stop_ms() * 1000.0 / (reps * copies)
    del bufs
    return us


def bench_decode(ctx, torch, vxm, layers, n_layers, copies, ctx0, steps, warmup, mode, synced=False):
    """Decode `steps` tokens from context ctx0, rotating over `copies` weight copies.  synced: after
    every token the hidden state is copied to the host (vxm_memcpy_d2h, which waits for it), the one
    read-back per step that the reference's synchronous graph call implies."""
    import numpy as np
    cfg = dict(hidden_size=H, n_layers=n_layers, n_heads=NH, n_kv_heads=NKV, head_dim=HD, intermediate_size=F,
               rms_norm_eps=1e-6, rope_theta=10000)
    fn = vxm.host_randn(11, H, 1.0, 0.02)
    models = [vxm.MiniCPM4(ctx, cfg, layers, final_norm=fn) for _ in range(copies)]
    for m in models:
        m.set_decode_mode(mode)
    cap = 1024
    kv = vxm.KVCache(ctx, n_layers, NKV, HD, cap)
    kv_prefill(vxm, kv, n_layers, ctx0, 5)
    x = torch.from_numpy(vxm.host_randn(3, H, 0.0, 1.0).reshape(1, H)).to("cuda:0")
    # warmup tokens, then rewind the cache to ctx0
    for i in range(warmup):
        models[i % copies].forward(kv, x, ctx0 + i)
    ctx.sync()
    kv.set_used(ctx0)
    host = np.empty(H if n_layers else 1, np.float32)
    L_ = vxm.lib()
    t = Timer(torch, ctx)
    t.start()
    for i in range(steps):
        models[i % copies].forward(kv, x, ctx0 + i)
        if synced:
            ctx.check(L_.vxm_memcpy_d2h(ctx.h, host.ctypes.data_as(vxm.C.c_void_p), vxm._ptr(x), host.nbytes))
    ms = t.stop_ms()
    for m in models:
        m.check()
    ok = bool(torch.isfinite(x).all().item())
    kv.free()
    for m in models:
        m.free()
    return ms * 1000.0 / steps, ok


def bench_decode_long(ctx, torch, vxm, layers, copies, contexts, steps, mode):
    """28-layer decode at long contexts: one cache of capacity max(contexts) + steps filled once,
    `steps` tokens timed from each context.  Returns {context: us per token}."""
    cfg = dict(hidden_size=H, n_layers=L, n_heads=NH, n_kv_heads=NKV, head_dim=HD, intermediate_size=F,
               rms_norm_eps=1e-6, rope_theta=10000)
    fn = vxm.host_randn(11, H, 1.0, 0.02)
    models = [vxm.MiniCPM4(ctx, cfg, layers, final_norm=fn) for _ in range(copies)]
    for m in models:
        m.set_decode_mode(mode)
    warm = max(24, copies)
    kv = vxm.KVCache(ctx, L, NKV, HD, max(contexts) + max(steps, warm))
    kv_prefill(vxm, kv, L, max(contexts), 5)
    x = torch.from_numpy(vxm.host_randn(3, H, 0.0, 1.0).reshape(1, H)).to("cuda:0")
    out = {}
    for c0 in contexts:
        kv.set_used(c0)
        # every copy decodes before the timed tokens (its first call sets up its launch state), 24
        # tokens in all: after the host-side cache fill the first timed context otherwise ran at
        # 1.5x its steady per-token time (the GPU had been idle)
        for i in range(warm):
            models[i % copies].forward(kv, x, c0 + i)
        ctx.sync()
        kv.set_used(c0)
        t = Timer(torch, ctx)
        t.start()
        for i in range(steps):
            models[i % copies].forward(kv, x, c0 + i)
        out[c0] = t.stop_ms() * 1000.0 / steps
    for m in models:
        m.check()
    kv.free()
    for m in models:
        m.free()
    return out


def bench_gemm(ctx, torch, vxm, N, K, M, reps):
    """One Q8_0 x Q8_0 matmul of M activation rows (the MFMA GEMM), back to back."""
    import numpy as np

    w32 = vxm.host_randn(7, N * K, 0.0, 0.02).reshape(N, K)
    x = vxm.host_randn(8, M * K, 0.0, 1.0).reshape(M, K)
    w = ctx.upload_q8_0(vxm.host_quantize_q8_0(w32), N, K)
    xq, xs = ctx.quantize_q8_0(torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0"), vxm.QUANT_X86)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
    L_ = vxm.lib()
    a = (w.h, vxm._ptr(xq), vxm._ptr(xs), vxm._ptr(y))
    for _ in range(3):
        L_.vxm_mul_mat_q8_0_q8_0(ctx.h, a[0], a[1], a[2], M, a[3])
    ctx.sync()
    t = Timer(torch, ctx)
    t.start()
    for _ in range(reps):
        L_.vxm_mul_mat_q8_0_q8_0(ctx.h, a[0], a[1], a[2], M, a[3])
    us = t.stop_ms() * 1000.0 / reps
    w.free()
    return us


def prefill_ops(M, n_layers=L):
    """int8 multiply-adds x 2 of the Q8_0 GEMMs and f32 attention flops of an M-token causal prefill."""
    qd, kvd = NH * HD, NKV * HD
    weights = qd * H + 2 * kvd * H + H * qd + 2 * F * H + H * F
    gemm = 2 * M * weights * n_layers
    pairs = M * (M + 1) // 2
    attn = 2 * 2 * pairs * NH * HD * n_layers
    return gemm, attn


def bench_prefill(ctx, torch, vxm, layers, n_layers, M, reps):
    """M-token causal prefill of the stack from position 0 (vxm_minicpm4_forward)."""
    cfg = dict(hidden_size=H, n_layers=n_layers, n_heads=NH, n_kv_heads=NKV, head_dim=HD, intermediate_size=F,
               rms_norm_eps=1e-6, rope_theta=10000)
    fn = vxm.host_randn(11, H, 1.0, 0.02)
    m = vxm.MiniCPM4(ctx, cfg, layers, final_norm=fn)
    kv = vxm.KVCache(ctx, n_layers, NKV, HD, M)
    x0 = torch.from_numpy(vxm.host_randn(4, M * H, 0.0, 1.0).reshape(M, H)).to("cuda:0")
    x = x0.clone()
    m.forward(kv, x, 0)
    ctx.sync()
    t = Timer(torch, ctx)
    ms = 0.0
    for _ in range(reps):
        x.copy_(x0)
        torch.cuda.synchronize()
        t.start()
        m.forward(kv, x, 0)
        ms += t.stop_ms()
    ok = bool(torch.isfinite(x).all().item())
    kv.free()
    m.free()
    return ms * 1000.0 / reps, ok


DIT = dict(H=1024, L=12, NH=16, NKV=16, HD=64, F=4096, FEAT=64, P=4, PC=17)
# the reference's own LocDiT (src/gen_init.c:280-283,424-441): 16 query / 2 KV heads of 128, and per CFG
# branch mu (2) + t (1) + the previous patch as cond (4) + the latent patch (4) = 11 rows
DIT_REF = dict(H=1024, L=12, NH=16, NKV=2, HD=128, F=4096, FEAT=64, P=4, PC=4)


def make_locdit(vxm, seed, d=DIT):
    """Seeded synthetic LocDiT (hidden 1024, 12 blocks, FFN 4096, the heads of d), Q8_0 N(0, 0.02)."""
    H, F, FEAT, NHD, KVD = d["H"], d["F"], d["FEAT"], d["NH"] * d["HD"], d["NKV"] * d["HD"]
    off = [0]

    def q8(n, k):
        w = vxm.host_randn(seed, n * k, 0.0, 0.02, offset=off[0]).reshape(n, k)
        off[0] += n * k
        return vxm.host_quantize_q8_0(w)

    def vec(n, mean=0.0, std=0.02):
        v = vxm.host_randn(seed, n, mean, std, offset=off[0])
        off[0] += n
        return v

    layers = [dict(q_proj=q8(NHD, H), k_proj=q8(KVD, H), v_proj=q8(KVD, H), o_proj=q8(H, NHD),
                   gate_proj=q8(F, H), up_proj=q8(F, H), down_proj=q8(H, F), input_layernorm=vec(H, 1.0),
                   post_attention_layernorm=vec(H, 1.0)) for _ in range(d["L"])]
    w = dict(layers=layers, in_proj=q8(H, FEAT), in_bias=vec(H), cond_proj=q8(H, FEAT), cond_bias=vec(H),
             out_proj=q8(FEAT, H), out_bias=vec(FEAT), norm=vec(H, 1.0), t_w1=q8(H, H), t_w2=q8(H, H),
             dt_w1=q8(H, H), dt_w2=q8(H, H), t_b1=vec(H), t_b2=vec(H), dt_b1=vec(H), dt_b2=vec(H))
    cfg = dict(hidden_size=H, n_layers=d["L"], n_heads=d["NH"], n_kv_heads=d["NKV"], head_dim=d["HD"],
               intermediate_size=F, feat_dim=FEAT, cond_dim=FEAT, rms_norm_eps=1e-6, rope_theta=10000)
    return cfg, w


def locdit_eval_bytes(d=DIT):
    """Q8_0 bytes of one LocDiT evaluation: 12 blocks + in/out/cond projections."""
    H, F, FEAT, NHD, KVD = d["H"], d["F"], d["FEAT"], d["NH"] * d["HD"], d["NKV"] * d["HD"]
    blk = q8_bytes(NHD + 2 * KVD, H) + q8_bytes(H, NHD) + 2 * q8_bytes(F, H) + q8_bytes(H, F)
    return d["L"] * blk + 2 * q8_bytes(H, FEAT) + q8_bytes(FEAT, H)


BLOCK_MODES = {"auto": 0, "kernels": 1, "persistent": 2}   # vxm_locdit_set_block_mode


def bench_cfm(ctx, torch, vxm, reps, n_steps=10, d=DIT, schedule=None, blocks="auto"):
    """CFM solves: n_steps Euler steps (uniform unless schedule says otherwise), CFG 2.0 with CFG-Zero*
    (both branches in one batch of 2 x (3 + PC + P) rows per LocDiT evaluation), latent P x 64, PC cond
    tokens; blocks: the block strategy (launch by launch, one persistent launch, or the library's pick)."""
    cfg, w = make_locdit(vxm, 21, d)
    m = vxm.LocDiT(ctx, cfg, w)
    m.set_block_mode(BLOCK_MODES[blocks])
    P, PC, H, FEAT = d["P"], d["PC"], d["H"], d["FEAT"]
    schedule = vxm.CFM_UNIFORM if schedule is None else schedule
    x0 = torch.from_numpy(vxm.host_randn(22, P * FEAT).reshape(P, FEAT)).to("cuda:0")
    cond = torch.from_numpy(vxm.host_randn(23, PC * FEAT).reshape(PC, FEAT)).to("cuda:0")
    mu = torch.from_numpy(vxm.host_randn(24, 2 * H).reshape(2, H)).to("cuda:0")
    x = x0.clone()
    # two untimed solves: the first runs eagerly, the second records the Euler loop as a graph
    for _ in range(2):
        x.copy_(x0)
        m.cfm_solve(x, cond, mu, n_steps, 2.0, schedule, True)
    ctx.sync()
    t = Timer(torch, ctx)
    ms = 0.0
    for _ in range(reps):
        x.copy_(x0)
        torch.cuda.synchronize()
        t.start()
        m.cfm_solve(x, cond, mu, n_steps, 2.0, schedule, True)
        ms += t.stop_ms()
    ok = bool(torch.isfinite(x).all().item())
    m.free()
    evals = n_steps - vxm.host_cfm_zero_star_steps(n_steps)
    return ms * 1000.0 / reps, evals, ok


# the per-token LM update: LocEnc (hidden 1024, 12 bidirectional blocks, 16 / 2 heads x 128, FFN 4096,
# one 4-position latent patch + the special token), the TSLM above, an 8-layer RALM of the same block
# shape without rope, FSQ 2048 -> 512 -> 2048 and the fusion projection 4096 -> 2048
ENC = dict(H=1024, L=12, NH=16, NKV=2, HD=128, F=4096, FEAT=64, P=4)
RALM_L, FSQ_DIM = 8, 512


def lm_update_bytes(ctx_len):
    """Algorithmic HBM bytes of one LM update: every weight once, gains, both LMs' KV read + append."""
    e = ENC
    qd, kvd = e["NH"] * e["HD"], e["NKV"] * e["HD"]
    enc_blk = (q8_bytes(qd, e["H"]) + 2 * q8_bytes(kvd, e["H"]) + q8_bytes(e["H"], qd) + 2 * q8_bytes(e["F"], e["H"])
               + q8_bytes(e["H"], e["F"]) + 2 * e["H"] * 4)
    proj = (q8_bytes(e["H"], e["FEAT"]) + q8_bytes(H, e["H"]) + q8_bytes(FSQ_DIM, H) + q8_bytes(H, FSQ_DIM)
            + q8_bytes(H, 2 * H))
    return step_bytes(ctx_len) + step_bytes(ctx_len, RALM_L) + e["L"] * enc_blk + proj


def bench_lm_update(ctx, torch, vxm, tslm_layers, ctx0, steps, warmup, prompt_tokens=0):
    """gen_lm_update per generated patch: LocEnc + enc_to_lm, the 28-layer TSLM step, FSQ, the fusion
    projection and the 8-layer RALM step, one stream-ordered call per token."""
    e = ENC
    enc_layers = make_layers(vxm, 31, e["L"], e["H"], e["NH"], e["NKV"], e["HD"], e["F"])
    ralm_layers = make_layers(vxm, 32, RALM_L)
    off = [0]

    def q8(n, k):
        w = vxm.host_randn(33, n * k, 0.0, 0.02, offset=off[0]).reshape(n, k)
        off[0] += n * k
        return vxm.host_quantize_q8_0(w)

    def vec(n, mean=0.0, std=0.02):
        v = vxm.host_randn(33, n, mean, std, offset=off[0])
        off[0] += n
        return v

    enc = vxm.LocEnc(ctx, dict(hidden_size=e["H"], n_layers=e["L"], n_heads=e["NH"], n_kv_heads=e["NKV"],
                               head_dim=e["HD"], intermediate_size=e["F"], feat_dim=e["FEAT"], rms_norm_eps=1e-6,
                               rope_theta=10000),
                     dict(layers=enc_layers, in_proj=q8(e["H"], e["FEAT"]), in_bias=vec(e["H"]),
                          special_token=vec(e["H"], 0.0, 1.0), norm=vec(e["H"], 1.0)))
    cfg = dict(hidden_size=H, n_layers=L, n_heads=NH, n_kv_heads=NKV, head_dim=HD, intermediate_size=F,
               rms_norm_eps=1e-6, rope_theta=10000)
    tslm = vxm.MiniCPM4(ctx, cfg, tslm_layers, final_norm=vec(H, 1.0))
    ralm = vxm.MiniCPM4(ctx, dict(cfg, n_layers=RALM_L, no_rope=1), ralm_layers, final_norm=vec(H, 1.0))
    pw = dict(enc_to_lm=q8(H, e["H"]), enc_to_lm_bias=vec(H), fsq_in=q8(FSQ_DIM, H), fsq_in_bias=vec(FSQ_DIM),
              fsq_out=q8(H, FSQ_DIM), fsq_out_bias=vec(H), fusion_concat=q8(H, 2 * H))
    u = vxm.LMUpdate(ctx, dict(lm_hidden=H, enc_hidden=e["H"], fsq_dim=FSQ_DIM, res_hidden=H, fsq_quant_scale=9.0),
                     pw, enc, tslm, ralm)
    tkv = vxm.KVCache(ctx, L, NKV, HD, 1024)
    rkv = vxm.KVCache(ctx, RALM_L, NKV, HD, 1024)
    kv_prefill(vxm, tkv, L, ctx0, 5)
    kv_prefill(vxm, rkv, RALM_L, ctx0, 6)
    patch = torch.from_numpy(vxm.host_randn(34, e["P"] * e["FEAT"]).reshape(e["P"], e["FEAT"])).to("cuda:0")
    outs = [torch.empty(H, dtype=torch.float32, device="cuda:0") for _ in range(4)]
    for i in range(warmup):
        u.step(tkv, rkv, patch, ctx0 + i, *outs)
    ctx.sync()
    tkv.set_used(ctx0)
    rkv.set_used(ctx0)
    t = Timer(torch, ctx)
    t.start()
    for i in range(steps):
        u.step(tkv, rkv, patch, ctx0 + i, *outs)
    ms = t.stop_ms()
    tslm.check()
    ralm.check()
    ok = all(bool(torch.isfinite(o).all().item()) for o in outs)
    prompt = None
    if prompt_tokens:
        # gen_prompt_eval_range: the prompt through the TSLM, the fusion projection and the RALM
        n = prompt_tokens
        x0 = torch.from_numpy(vxm.host_randn(35, n * H, 0.0, 1.0).reshape(n, H)).to("cuda:0")
        x = x0.clone()
        rh = torch.empty((n, H), dtype=torch.float32, device="cuda:0")
        u.prompt_prefill(tkv, rkv, x, 0, rh)
        ctx.sync()
        pms = 0.0
        for _ in range(3):
            x.copy_(x0)
            torch.cuda.synchronize()
            t.start()
            u.prompt_prefill(tkv, rkv, x, 0, rh)
            pms += t.stop_ms()
        prompt = (pms * 1000.0 / 3, bool(torch.isfinite(x).all().item() and torch.isfinite(rh).all().item()))
    u.free()
    for o in (enc, tslm, ralm, tkv, rkv):
        o.free()
    return ms * 1000.0 / steps, ok, prompt


def host_cores():
    """CPUs this process may run on: the affinity mask, the cgroup v2 CPU quota (cpu.max) and
    OMP_NUM_THREADS, each as found; `usable` is the smallest of them."""
    info = {"os_cpu_count": os.cpu_count()}
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        info["affinity"] = os.cpu_count()
    quota = None
    try:
        q, per = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        info["cgroup_cpu_max"] = f"{q} {per}"
        if q != "max":
            quota = int(q) / int(per)
    except (OSError, ValueError):
        info["cgroup_cpu_max"] = None
    info["cgroup_cpus"] = round(quota, 2) if quota else None
    omp = os.environ.get("OMP_NUM_THREADS")
    info["omp_num_threads"] = int(omp) if omp and omp.isdigit() else None
    cands = [c for c in (info["affinity"], int(quota) if quota and quota >= 1 else None, info["omp_num_threads"])
             if c]
    info["usable"] = max(1, min(cands)) if cands else 1
    return info


def cpu_baseline(vxm, layers, n_layers, ctx0, tokens, threads):
    """The oracle's SIMD restatement of ggml's CPU Q8_0 decode (1 copy of weights)."""
    import ctypes as C

    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    base = C.CDLL(oracle.BASE_LIB)
    base.cb_set_threads.argtypes = [C.c_int]
    base.cb_isa.restype = C.c_int
    base.cb_minicpm4_forward.argtypes = [C.POINTER(oracle.Cfg), C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                         C.c_int64, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32]
    cfg = oracle.make_cfg(H, NH, NKV, HD, F, eps=1e-6, rope_theta=10000.0, rope_ff=oracle.ROPE_SHORT_FACTORS)
    lws = [oracle.LayerW(wq=d["q_proj"], wk=d["k_proj"], wv=d["v_proj"], wo=d["o_proj"], wg=d["gate_proj"],
                         wu=d["up_proj"], wd=d["down_proj"], g_in=d["input_layernorm"],
                         g_post=d["post_attention_layernorm"]) for d in layers[:n_layers]]
    arr = (oracle.Layer * n_layers)(*[l.struct() for l in lws])
    cap = ctx0 + tokens + 1
    rng = np.random.default_rng(5)
    kcs = [oracle.fp32_to_fp16_bits(rng.normal(0, 1, NKV * cap * HD).astype(np.float32)) for _ in range(n_layers)]
    vcs = [oracle.fp32_to_fp16_bits(rng.normal(0, 1, NKV * cap * HD).astype(np.float32)) for _ in range(n_layers)]
    kp = (C.c_void_p * n_layers)(*[k.ctypes.data for k in kcs])
    vp = (C.c_void_p * n_layers)(*[v.ctypes.data for v in vcs])
    fn = np.ones(H, np.float32)
    x = rng.normal(0, 1, H).astype(np.float32)
    base.cb_set_threads(threads)
    # one untimed token to warm caches / thread pool
    base.cb_minicpm4_forward(C.byref(cfg), C.cast(arr, C.c_void_p), n_layers, fn.ctypes.data, x.ctypes.data, 1,
                             C.cast(kp, C.c_void_p), C.cast(vp, C.c_void_p), cap, ctx0)
    t0 = time.perf_counter()
    for i in range(tokens):
        base.cb_minicpm4_forward(C.byref(cfg), C.cast(arr, C.c_void_p), n_layers, fn.ctypes.data, x.ctypes.data,
                                 1, C.cast(kp, C.c_void_p), C.cast(vp, C.c_void_p), cap, ctx0 + i)
    dt = time.perf_counter() - t0
    return dt * 1e6 / tokens, ("avx512-vnni" if base.cb_isa() else "avx2")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help="decode tokens timed (context 256 -> 256+steps)")
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--copies", type=int, default=3, help="rotated copies of the 28-layer weights")
    ap.add_argument("--mode", default="auto", choices=["auto", "kernels", "persistent"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-tokens", type=int, default=96, help="decode tokens timed on all host cores")
    ap.add_argument("--cpu-tokens-1t", type=int, default=16, help="decode tokens timed on one host core")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the 28-layer decode (for profiling the dominant kernel)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time only the prefill legs (MFMA GEMMs and the 512-token 28-layer prefill)")
    ap.add_argument("--prefill-tokens", type=int, default=512)
    ap.add_argument("--prefill-long-tokens", type=int, default=2048,
                    help="tokens of the long-prompt prefill leg (0: skip it)")
    ap.add_argument("--cfm-only", action="store_true", help="time only the CFM solve leg")
    ap.add_argument("--blocks", default="auto", choices=list(BLOCK_MODES),
                    help="LocDiT block strategy of the CFM legs (auto: the library's pick per shape)")
    ap.add_argument("--gemv-only", action="store_true", help="time only the isolated Q8_0 GEMV leg")
    ap.add_argument("--lm-update-only", action="store_true", help="time only the per-token LM update leg")
    ap.add_argument("--long-context-only", action="store_true",
                    help="time only the 28-layer decode at long contexts (single-launch and per-op paths)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 3 device copies of 256 MiB (a known-traffic kernel for HBM counter scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import vxm

    mode = {"auto": 0, "kernels": 1, "persistent": 2}[args.mode]
    if args.copy_calibration:
        a = torch.empty(64 << 20, dtype=torch.float32, device="cuda:0").fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 256 MiB device copies (read 256 MiB + write 256 MiB each)")
        del a, b
    ctx = vxm.Context(0)
    res = {}
    pre = None
    cfm = None
    if not (args.decode_only or args.prefill_only or args.gemv_only or args.lm_update_only or args.long_context_only):
        us_cfm, evals, fin = bench_cfm(ctx, torch, vxm, 5, blocks=args.blocks)
        eb = locdit_eval_bytes()
        ops = 2 * 2 * (3 + DIT["PC"] + DIT["P"]) * (eb * 32 // 34)
        cfm = {"us_per_solve": round(us_cfm, 1), "evals": evals, "us_per_eval": round(us_cfm / evals, 1),
               "weight_GBs": round(evals * eb / (us_cfm * 1e-6) / 1e9, 1),
               "int8_TOPs": round(evals * ops / (us_cfm * 1e-6) / 1e12, 2), "finite": fin,
               "blocks": args.blocks,
               "note": "10 uniform steps, CFG 2.0 + CFG-Zero* (first step skipped), both branches batched "
                       "(M = 2 x 24); weights 214 MB per evaluation, Infinity-Cache resident"}
        log(f"cfm solve: {us_cfm:.1f} us for {evals} evaluations ({us_cfm / evals:.1f} us each), "
            f"{cfm['weight_GBs']} GB/s of weights, finite={fin}")
        us_r, evals_r, fin_r = bench_cfm(ctx, torch, vxm, 5, 10, DIT_REF, vxm.CFM_SWAY, blocks=args.blocks)
        ebr = locdit_eval_bytes(DIT_REF)
        rows_r = 2 * (3 + DIT_REF["PC"] + DIT_REF["P"])
        cfm["reference_shape"] = {
            "us_per_solve": round(us_r, 1), "evals": evals_r, "us_per_eval": round(us_r / evals_r, 1),
            "weight_GBs": round(evals_r * ebr / (us_r * 1e-6) / 1e9, 1),
            "int8_TOPs": round(evals_r * 2 * rows_r * (ebr * 32 // 34) / (us_r * 1e-6) / 1e12, 2), "finite": fin_r,
            "note": "the reference's LocDiT: 16 q / 2 kv heads x 128, 2 x 11 rows, 10 sway steps, CFG 2.0 + "
                    f"CFG-Zero*; weights {ebr / 1e6:.0f} MB per evaluation"}
        log(f"cfm solve, reference shape: {us_r:.1f} us for {evals_r} evaluations ({us_r / evals_r:.1f} us each), "
            f"finite={fin_r}")
        if args.cfm_only:
            print(json.dumps({"cfm": cfm}))
            ctx.close()
            return
    if not (args.decode_only or args.gemv_only or args.lm_update_only or args.long_context_only):
        M = args.prefill_tokens
        gemms = {}
        for name, (N, K) in (("qkv", (NH * HD + 2 * NKV * HD, H)), ("o", (H, NH * HD)), ("gate_up", (2 * F, H)),
                             ("down", (H, F))):
            us = bench_gemm(ctx, torch, vxm, N, K, M, 20)
            tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
            gemms[name] = {"N": N, "K": K, "M": M, "us": round(us, 2), "TOPs": round(tops, 1),
                           "mfma_frac": round(tops / INT8_PEAK_TOPS, 4)}
            log(f"gemm {name} {N}x{K} M={M}: {us:.2f} us, {tops:.1f} TOP/s ({100 * tops / INT8_PEAK_TOPS:.1f}% int8)")
        t0 = time.time()
        pl = make_layers(vxm, 1, L)
        log(f"generated {L} Q8_0 layers in {time.time() - t0:.1f} s")
        us_pre, fin = bench_prefill(ctx, torch, vxm, pl, L, M, 3)
        g_ops, a_flops = prefill_ops(M)
        pre = {"tokens": M, "layers": L, "us": round(us_pre, 1), "tokens_per_s": round(M / (us_pre * 1e-6), 1),
               "gemm_TOPs": round(g_ops / (us_pre * 1e-6) / 1e12, 1),
               "gemm_mfma_frac_of_step": round(g_ops / (us_pre * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4),
               "attention_GFLOP": round(a_flops / 1e9, 2), "finite": fin, "gemm": gemms}
        log(f"prefill {M} tokens x {L} layers: {us_pre:.1f} us ({M / (us_pre * 1e-6):.0f} tok/s), "
            f"GEMM work {g_ops / (us_pre * 1e-6) / 1e12:.1f} TOP/s over the step, finite={fin}")
        if args.prefill_long_tokens > 0:
            # a long prompt: spans past one 512-key score tile take the three-pass MFMA attention
            ML = args.prefill_long_tokens
            us_l, fin_l = bench_prefill(ctx, torch, vxm, pl, L, ML, 2)
            g_l, a_l = prefill_ops(ML)
            pre["long_prompt"] = {"tokens": ML, "layers": L, "us": round(us_l, 1),
                                  "tokens_per_s": round(ML / (us_l * 1e-6), 1),
                                  "gemm_TOPs": round(g_l / (us_l * 1e-6) / 1e12, 1),
                                  "attention_GFLOP": round(a_l / 1e9, 2), "finite": fin_l}
            log(f"prefill {ML} tokens x {L} layers: {us_l:.1f} us ({ML / (us_l * 1e-6):.0f} tok/s), finite={fin_l}")
        del pl
        if args.prefill_only:
            print(json.dumps({"prefill": pre}))
            ctx.close()
            return
    if not (args.decode_only or args.lm_update_only or args.long_context_only):
        for (N, K) in ((6144, 2048), (2048, 6144)):
            gb = gemv_bytes(N, K)
            us = bench_gemv(ctx, torch, vxm, N, K, 64, 10)
            gbs = gb / (us * 1e-6) / 1e9
            us_m, same = bench_gemv_multi(ctx, torch, vxm, N, K, 64, 10)
            mgbs = 64 * gb / (us_m * 1e-6) / 1e9
            rus1 = bench_read_floor(ctx, torch, vxm, gb, 64, 10, 1)
            rus64 = bench_read_floor(ctx, torch, vxm, gb, 64, 10, 64)
            res[f"{N}x{K}"] = {"us_per_launch": round(us, 3), "GBs": round(gbs, 1),
                               "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                               "read_floor_us_per_launch": round(rus1, 3),
                               "read_floor_GBs": round(gb / (rus1 * 1e-6) / 1e9, 1),
                               "multi": {"gemvs_per_launch": 64, "us_per_launch": round(us_m, 2),
                                         "us_per_gemv": round(us_m / 64, 3), "GBs": round(mgbs, 1),
                                         "hbm_frac": round(mgbs / HBM_PEAK_GBS, 4),
                                         "bit_identical_to_single": same,
                                         "read_floor_GBs": round(gb / (rus64 * 1e-6) / 1e9, 1),
                                         "read_floor_hbm_frac": round(gb / (rus64 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
                               "note": "us_per_launch: one launch per GEMV, back to back over 64 rotated weight "
                                       "copies (855 MB, beyond the 256 MB Infinity Cache); multi: the 64 copies "
                                       "in one launch; read_floor: vxm_stream_read of the same bytes, one buffer "
                                       "per launch / 64 per launch"}
            log(f"gemv {N}x{K}: {us:.3f} us/launch, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM); "
                f"64 per launch {us_m / 64:.3f} us/GEMV, {mgbs:.1f} GB/s ({100 * mgbs / HBM_PEAK_GBS:.1f}%), "
                f"bit-identical={same}; read floor {gb / (rus1 * 1e-6) / 1e9:.1f} GB/s single, "
                f"{gb / (rus64 * 1e-6) / 1e9:.1f} GB/s 64 per launch")
        if args.gemv_only:
            print(json.dumps({"gemv": res}))
            ctx.close()
            return

    t0 = time.time()
    layers = make_layers(vxm, 1, L)
    log(f"generated {L} Q8_0 layers in {time.time() - t0:.1f} s")

    us1 = None
    if not (args.decode_only or args.lm_update_only or args.long_context_only):
        # one decoder layer, context 512 (8 rotated copies of the layer)
        # 200 untimed tokens (about 10 ms): with 4, the GPU's clocks had not come up after the
        # previous leg's host work and the leg read 52-123 us from run to run
        us1, _ = bench_decode(ctx, torch, vxm, layers[:1], 1, 8, 512, 64, 200, mode)
        layer_b = step_bytes(512, 1)
        log(f"one layer decode @ctx512: {us1:.2f} us, {layer_b / (us1 * 1e-6) / 1e9:.1f} GB/s")

    longc = None
    if args.long_context_only or not (args.decode_only or args.lm_update_only):
        contexts = (1024, 2048, 4096, 8000) if args.long_context_only else (4096, 8000)
        lc = bench_decode_long(ctx, torch, vxm, layers, args.copies, contexts, 16, 2)
        longc = {"contexts": {str(c): {"us_per_token": round(u, 1),
                                       "GBs": round(step_bytes(c + 7.5) / (u * 1e-6) / 1e9, 1)}
                              for c, u in lc.items()},
                 "note": f"single-launch decode, 16 tokens from each context after 24 untimed ones, cache capacity "
                         f"{max(contexts) + 24}; "
                         "the keys of each head are split over up to 16 workgroups beyond 384"}
        log("long-context decode (single launch): " +
            ", ".join(f"ctx {c} {u:.1f} us" for c, u in lc.items()))
        if args.long_context_only:
            lk = bench_decode_long(ctx, torch, vxm, layers, args.copies, contexts, 8, 1)
            longc["per_op_us_per_token"] = {str(c): round(u, 1) for c, u in lk.items()}
            log("long-context decode (per-op kernels): " +
                ", ".join(f"ctx {c} {u:.1f} us" for c, u in lk.items()))
            print(json.dumps({"long_context": longc}))
            ctx.close()
            return

    mean_ctx = 256 + (args.steps - 1) / 2.0
    if args.lm_update_only:
        us_u, fin_u, _ = bench_lm_update(ctx, torch, vxm, layers, 256, args.steps, args.warmup)
        log(f"lm update (LocEnc + TSLM + FSQ + RALM): {us_u:.1f} us/token, finite={fin_u}")
        print(json.dumps({"lm_update": {"us_per_update": round(us_u, 1), "finite": fin_u}}))
        ctx.close()
        return
    us_step, finite = bench_decode(ctx, torch, vxm, layers, L, args.copies, 256, args.steps, args.warmup, mode)
    sb = step_bytes(mean_ctx)
    gbs = sb / (us_step * 1e-6) / 1e9
    log(f"28-layer decode step: {us_step:.1f} us/token, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% HBM), "
        f"finite={finite}")
    us_sync, _ = bench_decode(ctx, torch, vxm, layers, L, args.copies, 256, args.steps, args.warmup, mode, synced=True)
    log(f"28-layer decode step with one host read-back per token: {us_sync:.1f} us/token")
    lmu = None
    if not args.decode_only:
        us_u, fin_u, prm = bench_lm_update(ctx, torch, vxm, layers, 256, args.steps, args.warmup,
                                           prompt_tokens=args.prefill_tokens)
        ub = lm_update_bytes(mean_ctx)
        lmu = {"us_per_update": round(us_u, 1), "bytes": int(ub), "GBs": round(ub / (us_u * 1e-6) / 1e9, 1),
               "hbm_frac": round(ub / (us_u * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "finite": fin_u,
               "note": f"LocEnc 12 x hidden 1024 on a 4-position patch + 28-layer TSLM step + FSQ 512 + fusion + "
                       f"{RALM_L}-layer RALM step, ctx 256->{256 + args.steps}, one call per token, no host sync"}
        log(f"lm update (LocEnc + TSLM + FSQ + RALM): {us_u:.1f} us/token, {lmu['GBs']} GB/s, finite={fin_u}")
        if prm:
            lmu["prompt_prefill"] = {"tokens": args.prefill_tokens, "us": round(prm[0], 1),
                                     "tokens_per_s": round(args.prefill_tokens / (prm[0] * 1e-6), 1),
                                     "finite": prm[1],
                                     "note": "gen_prompt_eval_range: 28-layer TSLM + fusion_concat (4096 -> 2048) + "
                                             f"{RALM_L}-layer RALM over the prompt, one stream-ordered call"}
            log(f"prompt prefill ({args.prefill_tokens} tokens, TSLM + fusion + RALM): {prm[0]:.1f} us, "
                f"finite={prm[1]}")
    ctx.close()

    cpu = None
    if not args.no_cpu:
        cores = host_cores()
        threads = cores["usable"]
        t0 = time.time()
        c1, isa = cpu_baseline(vxm, layers, L, 256, args.cpu_tokens_1t, 1)
        cn, _ = cpu_baseline(vxm, layers, L, 256, args.cpu_tokens, threads)
        log(f"cpu baseline: 1 thread {c1 / 1000:.1f} ms/token, {threads} threads {cn / 1000:.1f} ms/token ({isa}), "
            f"{time.time() - t0:.1f} s")
        cpu = {"value": round(sb / (cn * 1e-6) / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{args.cpu_tokens} decode tokens on {threads} threads and {args.cpu_tokens_1t} on 1 thread "
                         f"of the 28-layer stack at context 256 (SIMD {isa} restatement of ggml-cpu's Q8_0 "
                         f"mul_mat path, one copy of the weights)",
               "host": cores,
               "us_per_step": round(cn, 1), "us_per_step_1thread": round(c1, 1),
               "thread_scaling": round(c1 / cn, 2),
               "speedup_vs_cpu_all_cores": round(cn / us_step, 1),
               "speedup_vs_cpu_1thread": round(c1 / us_step, 1)}

    # roofline of the dominant kernel: the persistent decode (one launch per
    # token step); its per-launch time is the timed region over the launches
    kname = ("k_decode_persistent<Shape<2048,16,2,128,6144>>" if args.mode != "kernels"
             else "per-op kernel sequence (no single dominant launch)")
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic() if args.mode != "kernels" else None, "kernel": kname,
            "bytes_per_launch": int(sb), "us_per_launch": round(us_step, 2)}

    out = {
        "metric": "Q8_0 decode GEMV GB/s (% HBM peak) + us per 28-layer decode step, 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1000.0, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"28-layer MiniCPM4 decode, batch 1, hidden 2048, 16/2 heads x 128, FFN 6144, "
                               f"Q8_0 N(0,0.02) seed 1, f16 KV ctx 256->{256 + args.steps} ({args.steps} tokens "
                               f"timed), {args.copies} rotated weight copies",
                   "decode_mode": args.mode, "context_start": 256, "context_end": 256 + args.steps},
        "us_per_step": round(us_step, 2),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "decode_synced": {"us_per_step": round(us_sync, 2),
                          "note": "the same tokens with the 8 KB hidden state copied to the host after each one "
                                  "(vxm_memcpy_d2h, which waits for it), the read-back per step of the reference's "
                                  "synchronous vcpm_backend_compute_graph"},
        "step_bytes": int(sb),
        "gemv": res,
        "layer_decode_ctx512_us": round(us1, 3) if us1 is not None else None,
        "prefill": pre,
        "cfm": cfm,
        "lm_update": lmu,
        "long_context": longc,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
