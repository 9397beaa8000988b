"""Float64 numpy decoder: an independent forward pass for pinning the oracle.

Vectorised restatement of the decoder the reference runs
(src/lib/llama-wgsl-runtime.ts:1025-1150): llama/qwen3 layers
(pre-norm, GQA attention with optional per-head q/k RMSNorm, RoPE interleaved
for GGUF arch "llama" and split-half otherwise, SwiGLU) and gemma3 layers
(sandwich norms, +-65000 residual clamp, GELU-tanh, sqrt(hidden) embedding
scale, sliding window on layers i % 6 != 5) and openelm layers (one fused
q|k|v matrix, per-layer head / kv-head / feed-forward counts from metadata
arrays, q/k RMSNorm, split-half RoPE). Everything is float64 except the
dequantized weights (exact float32 values) and, optionally, a binary16 K/V
cache. Closed forms only: no reduction-order mimicry.
"""
from __future__ import annotations

import numpy as np

from .ggufpy import Gguf, matrix, read_gguf


class NumpyDecoder:
    def __init__(self, path: str, vocab: int, max_context: int, kv_f16: bool = False):
        g: Gguf = read_gguf(path)
        self.g = g
        arch = g.kv["general.architecture"]
        self.arch = arch
        self.gemma = arch == "gemma3"
        self.interleaved = arch == "llama"
        p = arch + "."
        self.L = int(g.kv[p + "block_count"])
        self.H = int(g.kv[p + "embedding_length"])
        self.openelm = arch == "openelm"
        hc, kvc = g.kv[p + "attention.head_count"], g.kv[p + "attention.head_count_kv"]
        self.lnh = [int(x) for x in hc] if self.openelm else [int(hc)] * self.L
        self.lnkv = [int(x) for x in kvc] if self.openelm else [int(kvc)] * self.L
        self.nh, self.nkv = max(self.lnh), max(self.lnkv)
        self.hd = int(g.kv.get(p + "attention.key_length", self.H // self.nh))
        self.eps = float(np.float32(g.kv.get(p + "attention.layer_norm_rms_epsilon", 1e-5)))
        self.vocab = vocab
        self.ctx = min(max_context, int(g.kv.get(p + "context_length", max_context)))
        self.kv_f16 = kv_f16
        if self.gemma:
            gtheta = g.kv.get("gemma3.rope.freq_base", 1e6)
            win = int(g.kv.get("gemma3.attention.sliding_window", 0))
            self.theta = [round(gtheta) if i % 6 == 5 else 10000 for i in range(self.L)]
            self.window = [0 if i % 6 == 5 else win for i in range(self.L)]
        else:
            self.theta = [round(g.kv.get(p + "rope.freq_base", 10000.0))] * self.L
            self.window = [0] * self.L
        self.qk_norm = "blk.0.attn_q_norm.weight" in g.tensors
        self.emb = matrix(g, "token_embd.weight").astype(np.float64)
        self.lm = (matrix(g, "output.weight") if "output.weight" in g.tensors else self.emb).astype(np.float64)
        self.final_norm = matrix(g, "output_norm.weight").astype(np.float64)
        self.layers = []
        for i in range(self.L):
            b = f"blk.{i}."
            get = lambda n: matrix(g, b + n).astype(np.float64)
            if self.openelm:
                qkv = get("attn_qkv.weight")
                qd, kd = self.lnh[i] * self.hd, self.lnkv[i] * self.hd
                lay = dict(q=qkv[:qd], k=qkv[qd:qd + kd], v=qkv[qd + kd:qd + 2 * kd])
            else:
                lay = dict(q=get("attn_q.weight"), k=get("attn_k.weight"), v=get("attn_v.weight"))
            lay.update(o=get("attn_output.weight"), gate=get("ffn_gate.weight"), up=get("ffn_up.weight"),
                       down=get("ffn_down.weight"), in_norm=get("attn_norm.weight"))
            if self.gemma:
                lay.update(post=get("post_attention_norm.weight"), pre_ffn=get("ffn_norm.weight"),
                           post_ffn=get("post_ffw_norm.weight"))
            else:
                lay.update(post=get("ffn_norm.weight"))
            if self.qk_norm:
                lay.update(qn=get("attn_q_norm.weight"), kn=get("attn_k_norm.weight"))
            self.layers.append(lay)
        self.reset()

    def reset(self):
        self.pos = 0
        self.K = np.zeros((self.L, self.nkv, self.ctx, self.hd))
        self.V = np.zeros((self.L, self.nkv, self.ctx, self.hd))

    def _rms(self, x, w, eps=None):
        eps = self.eps if eps is None else eps
        return x / np.sqrt(np.mean(x * x) + eps) * w

    def _rope(self, x, theta):
        # x: [heads, hd]; rotate pairs
        half = self.hd // 2
        d = np.arange(half)
        ang = self.pos * np.power(float(theta), -2.0 * d / self.hd)
        co, si = np.cos(ang), np.sin(ang)
        y = x.copy()
        if self.interleaved:
            a, b = x[:, 0::2], x[:, 1::2]
            y[:, 0::2] = a * co - b * si
            y[:, 1::2] = a * si + b * co
        else:
            a, b = x[:, :half], x[:, half:]
            y[:, :half] = a * co - b * si
            y[:, half:] = a * si + b * co
        return y

    def step(self, token: int) -> np.ndarray:
        H, hd = self.H, self.hd
        x = self.emb[token] * (np.sqrt(H) if self.gemma else 1.0)
        if self.gemma:
            x = x * 1.0
        for i, lay in enumerate(self.layers):
            nh, nkv = self.lnh[i], self.lnkv[i]
            n = self._rms(x, lay["in_norm"])
            q = (lay["q"] @ n).reshape(nh, hd)
            k = (lay["k"] @ n).reshape(nkv, hd)
            v = (lay["v"] @ n).reshape(nkv, hd)
            if self.qk_norm:
                q = np.stack([self._rms(h, lay["qn"]) for h in q])
                k = np.stack([self._rms(h, lay["kn"]) for h in k])
            q = self._rope(q, self.theta[i])
            k = self._rope(k, self.theta[i])
            if self.kv_f16:
                k = k.astype(np.float16).astype(np.float64)
                v = v.astype(np.float16).astype(np.float64)
            self.K[i, :nkv, self.pos] = k
            self.V[i, :nkv, self.pos] = v
            w = self.window[i]
            start = self.pos + 1 - w if (w and self.pos + 1 > w) else 0
            grp = nh // nkv
            out = np.empty((nh, hd))
            for h in range(nh):
                kk = self.K[i, h // grp, start:self.pos + 1]
                vv = self.V[i, h // grp, start:self.pos + 1]
                s = kk @ q[h] / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                out[h] = p @ vv
            o = lay["o"] @ out.reshape(-1)
            if self.gemma:
                x = np.clip(x + self._rms(o, lay["post"]), -65000, 65000)
                n = self._rms(x, lay["pre_ffn"])
                gte = lay["gate"] @ n
                up = lay["up"] @ n
                c = 0.7978845608028654
                gelu = np.where(gte > 10, gte, np.where(gte < -10, 0.0,
                                0.5 * gte * (1 + np.tanh(c * (gte + 0.044715 * gte ** 3)))))
                d = lay["down"] @ (gelu * up)
                x = np.clip(x + self._rms(d, lay["post_ffn"]), -65000, 65000)
            else:
                x = x + o
                n = self._rms(x, lay["post"])
                gte = lay["gate"] @ n
                up = lay["up"] @ n
                x = x + lay["down"] @ (gte / (1 + np.exp(-gte)) * up)
        self.pos += 1
        self.last_hidden = x
        return self.lm[: self.vocab] @ self._rms(x, self.final_norm)


class NumpyGpt2:
    """Float64 GPT-2 decoder (the reference's GPT runtime, src/lib/gpt-wgsl-runtime.ts:749-840):
    token + learned position embedding; per layer LayerNorm -> fused q|k|v + bias ->
    multi-head attention -> output projection + bias -> residual, clamped to +-10000 (NaN -> 0);
    LayerNorm -> up + bias -> GELU-tanh -> down + bias -> residual, clamped; final LayerNorm ->
    output matrix. Closed forms in float64 (variance as the mean of squared deviations)."""

    def __init__(self, path: str, max_context: int, kv_f16: bool = False):
        g: Gguf = read_gguf(path)
        p = "gpt2."
        self.L = int(g.kv[p + "block_count"])
        self.H = int(g.kv[p + "embedding_length"])
        self.nh = int(g.kv[p + "attention.head_count"])
        self.hd = self.H // self.nh
        self.eps = float(np.float32(g.kv.get(p + "attention.layer_norm_epsilon", 1e-5)))
        self.ctx = min(max_context, int(g.kv[p + "context_length"]))
        self.kv_f16 = kv_f16
        f = lambda n: matrix(g, n).astype(np.float64)
        self.emb = f("token_embd.weight")
        self.vocab = self.emb.shape[0]
        self.pe = f("position_embd.weight")
        self.lm = f("output.weight")
        self.fn_w, self.fn_b = f("output_norm.weight"), f("output_norm.bias")
        self.layers = []
        for i in range(self.L):
            b = f"blk.{i}."
            self.layers.append({k: f(b + k) for k in (
                "attn_norm.weight", "attn_norm.bias", "attn_qkv.weight", "attn_qkv.bias", "attn_output.weight",
                "attn_output.bias", "ffn_norm.weight", "ffn_norm.bias", "ffn_up.weight", "ffn_up.bias",
                "ffn_down.weight", "ffn_down.bias")})
        self.reset()

    def reset(self):
        self.pos = 0
        self.K = np.zeros((self.L, self.nh, self.ctx, self.hd))
        self.V = np.zeros((self.L, self.nh, self.ctx, self.hd))

    def _ln(self, x, w, b):
        mu = x.mean()
        return (x - mu) / np.sqrt(((x - mu) ** 2).mean() + self.eps) * w + b

    @staticmethod
    def _gelu(x):
        c = 0.7978845608028654
        g = 0.5 * x * (1 + np.tanh(c * (x + 0.044715 * x ** 3)))
        return np.where(np.isnan(x), 0.0, np.where(x > 10, x, np.where(x < -10, 0.0, g)))

    @staticmethod
    def _sanitize(x):
        return np.where(np.isnan(x), 0.0, np.clip(x, -10000.0, 10000.0))

    def step(self, token: int) -> np.ndarray:
        H, hd, nh = self.H, self.hd, self.nh
        x = self.emb[token] + self.pe[self.pos]
        for i, lay in enumerate(self.layers):
            n = self._ln(x, lay["attn_norm.weight"], lay["attn_norm.bias"])
            qkv = lay["attn_qkv.weight"] @ n + lay["attn_qkv.bias"]
            q, k, v = qkv[:H].reshape(nh, hd), qkv[H:2 * H].reshape(nh, hd), qkv[2 * H:].reshape(nh, hd)
            if self.kv_f16:
                k = k.astype(np.float16).astype(np.float64)
                v = v.astype(np.float16).astype(np.float64)
            self.K[i, :, self.pos] = k
            self.V[i, :, self.pos] = v
            out = np.empty((nh, hd))
            for h in range(nh):
                s = self.K[i, h, :self.pos + 1] @ q[h] / np.sqrt(hd)
                pr = np.exp(s - s.max())
                out[h] = (pr / pr.sum()) @ self.V[i, h, :self.pos + 1]
            x = self._sanitize(x + lay["attn_output.weight"] @ out.reshape(-1) + lay["attn_output.bias"])
            n = self._ln(x, lay["ffn_norm.weight"], lay["ffn_norm.bias"])
            u = self._gelu(lay["ffn_up.weight"] @ n + lay["ffn_up.bias"])
            x = self._sanitize(x + lay["ffn_down.weight"] @ u + lay["ffn_down.bias"])
        self.pos += 1
        return self.lm @ self._ln(x, self.fn_w, self.fn_b)


class NumpyLfm2:
    """Float64 LFM2 decoder (the reference's LFM runtime, src/lib/lfm-wgsl-runtime.ts:727-809).

    Per layer: RMSNorm (eps 1e-5) -> either a gated short convolution
    (in_proj -> B, C, x; y_t = C * sum_j w_j (B*x)_{t-2+j} over the last three
    positions; out_proj) or GQA attention (q/k/v, per-head q/k RMSNorm, split-half
    RoPE with base 1e6, softmax(q.K / sqrt(hd)) V, output projection); residual;
    RMSNorm -> SwiGLU -> residual. Final RMSNorm (token_embd_norm) and the tied
    embedding as lm_head. A layer is a convolution layer when it holds
    shortconv.conv.weight. Closed forms in float64: the convolution is evaluated
    from a list of every position's B*x, not from a shifted state."""

    def __init__(self, path: str, vocab: int, max_context: int, kv_f16: bool = False):
        g: Gguf = read_gguf(path)
        p = "lfm2."
        self.L = int(g.kv[p + "block_count"])
        self.H = int(g.kv[p + "embedding_length"])
        self.nh = int(g.kv[p + "attention.head_count"])
        kv = g.kv[p + "attention.head_count_kv"]
        self.lnkv = [int(x) for x in kv] if isinstance(kv, (list, tuple)) else [int(kv)] * self.L
        self.hd = int(g.kv.get(p + "attention.key_length", self.H // self.nh))
        self.eps = 1e-5
        self.vocab = vocab
        self.ctx = max_context
        self.kv_f16 = kv_f16
        f = lambda n: matrix(g, n).astype(np.float64)
        self.emb = f("token_embd.weight")
        self.final_norm = f("token_embd_norm.weight")
        self.layers = []
        for i in range(self.L):
            b = f"blk.{i}."
            lay = dict(in_norm=f(b + "attn_norm.weight"), post=f(b + "ffn_norm.weight"), gate=f(b + "ffn_gate.weight"),
                       up=f(b + "ffn_up.weight"), down=f(b + "ffn_down.weight"))
            lay["conv"] = (b + "shortconv.conv.weight") in g.tensors
            if lay["conv"]:
                lay.update(w=f(b + "shortconv.conv.weight").reshape(self.H, 3), inp=f(b + "shortconv.in_proj.weight"),
                           out=f(b + "shortconv.out_proj.weight"))
            else:
                lay.update(q=f(b + "attn_q.weight"), k=f(b + "attn_k.weight"), v=f(b + "attn_v.weight"),
                           o=f(b + "attn_output.weight"), qn=f(b + "attn_q_norm.weight"),
                           kn=f(b + "attn_k_norm.weight"))
            self.layers.append(lay)
        self.reset()

    def reset(self):
        self.pos = 0
        self.K = [[] for _ in range(self.L)]
        self.V = [[] for _ in range(self.L)]
        self.bx = [[] for _ in range(self.L)]  # every position's B * x, per convolution layer

    def _rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.eps) * w

    def _rope(self, x):
        half = self.hd // 2
        ang = self.pos * np.power(1e6, -2.0 * np.arange(half) / self.hd)
        co, si = np.cos(ang), np.sin(ang)
        a, b = x[:, :half], x[:, half:]
        return np.concatenate([a * co - b * si, a * si + b * co], axis=1)

    def step(self, token: int) -> np.ndarray:
        H, hd = self.H, self.hd
        x = self.emb[token].copy()
        for i, lay in enumerate(self.layers):
            n = self._rms(x, lay["in_norm"])
            if lay["conv"]:
                pr = lay["inp"] @ n
                B, C, xx = pr[:H], pr[H:2 * H], pr[2 * H:]
                self.bx[i].append(B * xx)
                hist = ([np.zeros(H)] * 2 + self.bx[i])[-3:]  # positions t-2, t-1, t (zeros before 0)
                conv = sum(lay["w"][:, j] * hist[j] for j in range(3))
                o = lay["out"] @ (C * conv)
            else:
                nkv = self.lnkv[i]
                q = (lay["q"] @ n).reshape(self.nh, hd)
                k = (lay["k"] @ n).reshape(nkv, hd)
                v = (lay["v"] @ n).reshape(nkv, hd)
                q = self._rope(np.stack([self._rms(h, lay["qn"]) for h in q]))
                k = self._rope(np.stack([self._rms(h, lay["kn"]) for h in k]))
                if self.kv_f16:
                    k = k.astype(np.float16).astype(np.float64)
                    v = v.astype(np.float16).astype(np.float64)
                self.K[i].append(k)
                self.V[i].append(v)
                KK, VV = np.stack(self.K[i]), np.stack(self.V[i])  # [t, nkv, hd]
                grp = self.nh // nkv
                att = np.empty((self.nh, hd))
                for h in range(self.nh):
                    s = KK[:, h // grp] @ q[h] / np.sqrt(hd)
                    pw = np.exp(s - s.max())
                    att[h] = (pw / pw.sum()) @ VV[:, h // grp]
                o = lay["o"] @ att.reshape(-1)
            x = x + o
            n = self._rms(x, lay["post"])
            gte, up = lay["gate"] @ n, lay["up"] @ n
            x = x + lay["down"] @ (gte / (1 + np.exp(-gte)) * up)
        self.pos += 1
        self.last_hidden = x
        return self.emb[: self.vocab] @ self._rms(x, self.final_norm)


class NumpyGranite:
    """Float64 Granite-4.0-H decoder (the reference's Granite runtime,
    src/lib/granite-wgsl-runtime.ts:769-858).

    Embedding x12; per layer RMSNorm (eps 1e-5) -> either a Mamba2 block or NoPE
    GQA attention (scores x 1/64); residual += 0.246 * out; RMSNorm -> SwiGLU ->
    residual += 0.246 * out. Final RMSNorm, the tied embedding as lm_head, logits
    x 1/3. The Mamba2 block is evaluated in its dual (attention-like) form from
    the history of every position's (dt, B, x), not from a running state:
        y_t[n, h] = sum_{tau <= t} (C_t . B_tau) prod_{tau < u <= t} exp(dt_u[n] A[n])
                    * dt_tau[n] x_tau[n, h]  +  D[n] x_t[n, h],
    with the causal 4-tap convolution (+ bias, silu) over the history of xBC,
    then y * silu(z) through an RMSNorm over the inner size."""

    HDIM, STATE = 32, 128

    def __init__(self, path: str, max_context: int = 4096, kv_f16: bool = False):
        g: Gguf = read_gguf(path)
        f = lambda n: matrix(g, n).astype(np.float64)
        self.emb = f("token_embd.weight")
        self.H = self.emb.shape[1]
        self.final_norm = f("output_norm.weight")
        self.kv_f16 = kv_f16
        self.layers = []
        i = 0
        while f"blk.{i}.attn_norm.weight" in g.tensors:
            b = f"blk.{i}."
            lay = dict(in_norm=f(b + "attn_norm.weight"), post=f(b + "ffn_norm.weight"), gate=f(b + "ffn_gate.weight"),
                       up=f(b + "ffn_up.weight"), down=f(b + "ffn_down.weight"))
            lay["mamba"] = (b + "ssm_in.weight") in g.tensors
            if lay["mamba"]:
                lay.update(inp=f(b + "ssm_in.weight"), out=f(b + "ssm_out.weight"),
                           cw=f(b + "ssm_conv1d.weight").reshape(-1, 4), cb=f(b + "ssm_conv1d.bias"),
                           dtb=f(b + "ssm_dt.bias"), A=f(b + "ssm_a"), D=f(b + "ssm_d"), nw=f(b + "ssm_norm.weight"))
            else:
                lay.update(q=f(b + "attn_q.weight"), k=f(b + "attn_k.weight"), v=f(b + "attn_v.weight"),
                           o=f(b + "attn_output.weight"))
            self.layers.append(lay)
            i += 1
        self.reset()

    def reset(self):
        self.pos = 0
        self.K = [[] for _ in self.layers]
        self.V = [[] for _ in self.layers]
        self.xbc = [[] for _ in self.layers]   # every position's pre-convolution xBC
        self.hist = [[] for _ in self.layers]  # every position's (dt, B, x)

    @staticmethod
    def _rms(x, w):
        return x / np.sqrt(np.mean(x * x) + 1e-5) * w

    @staticmethod
    def _silu(x):
        return x / (1 + np.exp(-x))

    def _mamba(self, i, lay, n):
        inner = lay["out"].shape[1]
        nh, S = inner // self.HDIM, self.STATE
        pr = lay["inp"] @ n
        z, xbc, dtr = pr[:inner], pr[inner:inner + inner + 2 * S], pr[inner + inner + 2 * S:]
        self.xbc[i].append(xbc)
        win = ([np.zeros_like(xbc)] * 3 + self.xbc[i])[-4:]  # positions t-3 .. t (zeros before 0)
        conv = self._silu(sum(lay["cw"][:, j] * win[j] for j in range(4)) + lay["cb"])
        x, B, C = conv[:inner].reshape(nh, self.HDIM), conv[inner:inner + S], conv[inner + S:]
        sp = dtr + lay["dtb"]
        dt = np.where(sp > 20, sp + np.log1p(np.exp(-np.minimum(sp, 20.0))), np.log1p(np.exp(np.minimum(sp, 20.0))))
        self.hist[i].append((dt, B, x))
        y = lay["D"][:, None] * x
        logdecay = 0.0  # sum over u in (tau, t] of dt_u * A
        for dtt, Bt, xt in reversed(self.hist[i]):
            y = y + (C @ Bt) * (np.exp(logdecay) * dtt)[:, None] * xt
            logdecay = logdecay + dtt * lay["A"]
        g = y.reshape(-1) * self._silu(z)
        return lay["out"] @ self._rms(g, lay["nw"])

    def step(self, token: int) -> np.ndarray:
        hd = 64
        x = self.emb[token] * 12.0
        for i, lay in enumerate(self.layers):
            n = self._rms(x, lay["in_norm"])
            if lay["mamba"]:
                o = self._mamba(i, lay, n)
            else:
                nq, nkv = lay["q"].shape[0] // hd, lay["k"].shape[0] // hd
                q = (lay["q"] @ n).reshape(nq, hd)
                k = (lay["k"] @ n).reshape(nkv, hd)
                v = (lay["v"] @ n).reshape(nkv, hd)
                if self.kv_f16:
                    k = k.astype(np.float16).astype(np.float64)
                    v = v.astype(np.float16).astype(np.float64)
                self.K[i].append(k)
                self.V[i].append(v)
                KK, VV = np.stack(self.K[i]), np.stack(self.V[i])
                grp = nq // nkv
                att = np.empty((nq, hd))
                for h in range(nq):
                    s = KK[:, h // grp] @ q[h] * 0.015625
                    pw = np.exp(s - s.max())
                    att[h] = (pw / pw.sum()) @ VV[:, h // grp]
                o = lay["o"] @ att.reshape(-1)
            x = x + 0.246 * o
            n = self._rms(x, lay["post"])
            gte, up = lay["gate"] @ n, lay["up"] @ n
            x = x + 0.246 * (lay["down"] @ (self._silu(gte) * up))
        self.pos += 1
        self.last_hidden = x
        return (self.emb @ self._rms(x, self.final_norm)) / 3.0
