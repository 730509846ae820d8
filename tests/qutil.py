"""Low-bit weight helpers for the tests: ggml block quantizers (float
weights -> Q8_0 / Q4_K / Q5_K / Q6_K blocks, written from the published block
layouts, the inverse of oracle/ggml_quant.c's decoding; scale choices are
simple absmax / min-max ones, not llama.cpp's search) and a builder of
mixed-format Qwen3 weights for grout_engine_create_q together with the
matching oracle weights."""
import numpy as np

import oracle as O
from oracle import qwen3 as Q

F16 = 0
f32 = np.float32


def _safe(a):
    return np.where(a > 0, a, f32(1))


def quantize(fmt: int, w: np.ndarray) -> np.ndarray:
    """float [rows][k] -> uint8 ggml blocks [rows][k / block * bytes]."""
    w = np.asarray(w, f32)
    rows, k = w.shape
    if fmt == O.Q8_0:
        b = w.reshape(rows, k // 32, 32)
        d = (np.abs(b).max(-1) / f32(127)).astype(np.float16)
        df = d.astype(f32)
        q = np.clip(np.rint(b / _safe(df)[..., None]), -128, 127).astype(np.int8)
        out = np.zeros((rows, k // 32, 34), np.uint8)
        out[..., 0:2] = d.view(np.uint8).reshape(rows, k // 32, 2)
        out[..., 2:] = q.view(np.uint8)
        return out.reshape(rows, -1)
    nb = k // 256
    if fmt == O.Q6_K:
        b = w.reshape(rows, nb, 16, 16)  # 16 runs of 16 weights
        s = np.abs(b).max(-1) / f32(31)
        d = (s.max(-1) / f32(127)).astype(np.float16)
        df = d.astype(f32)
        sc = np.clip(np.rint(s / _safe(df)[..., None]), 0, 127).astype(np.int8)
        eff = df[..., None] * sc.astype(f32)
        q = np.clip(np.rint(b / _safe(eff)[..., None]) + 32, 0, 63)
        q = np.where(eff[..., None] > 0, q, 32).astype(np.uint8).reshape(rows, nb, 2, 4, 32)
        q1, q2, q3, q4 = (q[..., i, :] for i in range(4))  # weight 128 n + 32 i + l
        ql = np.empty((rows, nb, 2, 64), np.uint8)
        ql[..., :32] = (q1 & 0xF) | ((q3 & 0xF) << 4)
        ql[..., 32:] = (q2 & 0xF) | ((q4 & 0xF) << 4)
        qh = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
        out = np.zeros((rows, nb, 210), np.uint8)
        out[..., 0:128] = ql.reshape(rows, nb, 128)
        out[..., 128:192] = qh.reshape(rows, nb, 64)
        out[..., 192:208] = sc.view(np.uint8)
        out[..., 208:210] = d.view(np.uint8).reshape(rows, nb, 2)
        return out.reshape(rows, -1)
    if fmt in (O.Q4_K, O.Q5_K):
        qmax = 15 if fmt == O.Q4_K else 31
        b = w.reshape(rows, nb, 8, 32)  # 8 sub-blocks of 32 weights
        lo = np.minimum(b.min(-1), 0)
        scale = (b.max(-1) - lo) / f32(qmax)
        mn = -lo
        d = (scale.max(-1) / f32(63)).astype(np.float16)
        dmin = (mn.max(-1) / f32(63)).astype(np.float16)
        df, dmf = d.astype(f32), dmin.astype(f32)
        sc = np.clip(np.rint(scale / _safe(df)[..., None]), 0, 63).astype(np.int64)
        m = np.clip(np.rint(mn / _safe(dmf)[..., None]), 0, 63).astype(np.int64)
        es, em = df[..., None] * sc.astype(f32), dmf[..., None] * m.astype(f32)
        q = np.clip(np.rint((b + em[..., None]) / _safe(es)[..., None]), 0, qmax)
        q = np.where(es[..., None] > 0, q, 0).astype(np.uint8).reshape(rows, nb, 4, 2, 32)
        pk = np.zeros((rows, nb, 12), np.uint8)
        for j in range(4):  # 6-bit (scale, min) pairs in 12 bytes (get_scale_min_k4's inverse)
            pk[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
            pk[..., j + 4] = (m[..., j] & 63) | ((m[..., j + 4] >> 4) << 6)
            pk[..., j + 8] = (sc[..., j + 4] & 0xF) | ((m[..., j + 4] & 0xF) << 4)
        out = np.zeros((rows, nb, 144 if fmt == O.Q4_K else 176), np.uint8)
        out[..., 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
        out[..., 2:4] = dmin.view(np.uint8).reshape(rows, nb, 2)
        out[..., 4:16] = pk
        qs = ((q[..., 0, :] & 0xF) | ((q[..., 1, :] & 0xF) << 4)).reshape(rows, nb, 128)
        if fmt == O.Q4_K:
            out[..., 16:] = qs
        else:  # fifth bits: weight 64 g + l (+32) -> bit 2 g (2 g + 1) of qh[l]
            qh = np.zeros((rows, nb, 32), np.uint8)
            for g in range(4):
                qh |= ((q[..., g, 0, :] >> 4) << (2 * g)) | ((q[..., g, 1, :] >> 4) << (2 * g + 1))
            out[..., 16:48] = qh
            out[..., 48:] = qs
        return out.reshape(rows, -1)
    raise ValueError(f"format {fmt}")


class _Mat:
    """One matrix as the engine gets it and as the oracle multiplies it."""

    def __init__(self, fmt, w):
        rows, k = w.shape
        self.fmt = fmt
        if fmt == F16:
            self.gpu = w.astype(np.float16).view(np.uint16)
            self.f16 = self.gpu                     # prefill rows and decode
            self.dec = self.gpu.view(np.float16).astype(np.float64)
            self.cpu = self.gpu                     # embedding rows
        else:
            self.gpu = quantize(fmt, w)
            dec = O.dequant(fmt, self.gpu, rows * k, decode=True).reshape(rows, k)
            self.dec = dec.astype(np.float64)       # decode GEMV weights (fp32 values)
            self.f16 = dec.astype(np.float16).view(np.uint16)  # prefill dequant scratch
            self.cpu = O.dequant(fmt, self.gpu, rows * k).reshape(rows, k).astype(
                np.float16).view(np.uint16)         # embedding gather (CPU rule)


def mixed_weights(cfg, plan: dict, seed: int, std: float = 0.05):
    """plan: {"embed": fmt, "lm_head": fmt or None (tied),
    "layers": [{"q": fmt, "k", "v", "o", "gate", "up", "down"}, ...]}.
    Returns (QuantWeights keyword arguments, oracle host weights (fp16 bits),
    oracle decode_w64)."""
    rng = np.random.default_rng(seed)
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qd, kd = cfg.q_dim, cfg.kv_dim

    def mat(fmt, rows, k):
        return _Mat(fmt, (rng.standard_normal((rows, k)) * std).astype(f32))

    def vec(n):
        return rng.uniform(0.8, 1.2, n).astype(np.float16).view(np.uint16)

    embed = mat(plan["embed"], V, H)
    head = None if plan.get("lm_head") is None else mat(plan["lm_head"], V, H)
    gpu_layers, host_layers, w64 = [], [], {}
    for l, p in enumerate(plan["layers"]):
        m = {"q_proj": mat(p["q"], qd, H), "k_proj": mat(p["k"], kd, H),
             "v_proj": mat(p["v"], kd, H), "o_proj": mat(p["o"], H, qd),
             "gate_proj": mat(p["gate"], I, H), "up_proj": mat(p["up"], I, H),
             "down_proj": mat(p["down"], H, I)}
        v = {"input_layernorm": vec(H), "q_norm": vec(Q.D), "k_norm": vec(Q.D),
             "post_attention_layernorm": vec(H)}
        gl = dict(v)
        gl.update({k: (x.fmt, x.gpu) for k, x in m.items()})
        gpu_layers.append(gl)
        fused = {"qkv_proj": ("q_proj", "k_proj", "v_proj"), "o_proj": ("o_proj",),
                 "gate_up_proj": ("gate_proj", "up_proj"), "down_proj": ("down_proj",)}
        hl = dict(v)
        for key, names in fused.items():
            hl[key] = np.concatenate([m[n].f16 for n in names])
            w64[(l, key)] = np.concatenate([m[n].dec for n in names])
        host_layers.append(hl)
    w64["lm_head"] = (embed if head is None else head).dec
    norm = vec(H)
    spec = dict(embed_tokens=(embed.fmt, embed.gpu), norm=norm, layers=gpu_layers,
                lm_head=None if head is None else (head.fmt, head.gpu))
    host = dict(embed_tokens=embed.cpu, norm=norm, layers=host_layers,
                lm_head=None if head is None else head.f16)
    return spec, host, w64
