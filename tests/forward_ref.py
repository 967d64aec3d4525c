"""An fp64 forward pass written from the model's definition (not from the
oracle's code): dequantised weights (quant_ref), rmsnorm, rotary embedding
of adjacent pairs at theta^(-2i/d), grouped-query attention with softmax,
SiLU-gated FFN, residuals, final norm and classifier.  Used as a
mathematical pin of the oracle's forward and of the GPU's."""
import ast

import numpy as np

import quant_ref as Q


def model_from_golden(W, g, name):
    """Rebuild a golden forward case's tensors from its seeds."""
    spec = W.ModelSpec(*[int(v) for v in g["spec"]])
    salt, wt, et, ot = [int(v) for v in g[f"{name}_case"]]
    ov = dict(ast.literal_eval(str(g[f"{name}_overrides"])))
    t = W.make_model(spec, wt, salt=salt, embd_type=None if et < 0 else et,
                     output_type=None if ot < 0 else ot, overrides=ov)
    return spec, t


class Forward64:
    def __init__(self, spec, tensors):
        self.s = spec
        self.w = {}
        for name, (dims, ty, raw) in tensors.items():
            if len(dims) == 1:
                self.w[name] = np.asarray(raw, np.uint8).view(np.float32).astype(np.float64)
            else:
                cols, rows = dims
                self.w[name] = Q.dequant(np.asarray(raw, np.uint8), ty, rows, cols)
        if "output.weight" not in self.w:
            self.w["output.weight"] = self.w["token_embd.weight"]
        L, C, kv = spec.n_layers, spec.n_ctx, spec.kv_dim
        self.kc = np.zeros((L, C, kv))
        self.vc = np.zeros((L, C, kv))

    @staticmethod
    def rms(x, w, eps):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    def rope(self, x, pos):
        d = self.s.head_dim
        x = x.reshape(-1, d // 2, 2)
        i = np.arange(d // 2)
        ang = pos * self.s.rope_freq_base ** (-2.0 * i / d)
        c, s = np.cos(ang), np.sin(ang)
        out = np.empty_like(x)
        out[..., 0] = x[..., 0] * c - x[..., 1] * s
        out[..., 1] = x[..., 0] * s + x[..., 1] * c
        return out.reshape(-1)

    def forward(self, token, pos, silu_sign=1.0, residual=True):
        s, w, d = self.s, self.w, self.s.head_dim
        x = w["token_embd.weight"][token].copy()
        for l in range(s.n_layers):
            p = f"blk.{l}."
            xb = self.rms(x, w[p + "attn_norm.weight"], s.rms_norm_eps)
            q = self.rope(w[p + "attn_q.weight"] @ xb, pos)
            k = self.rope(w[p + "attn_k.weight"] @ xb, pos)
            v = w[p + "attn_v.weight"] @ xb
            self.kc[l, pos], self.vc[l, pos] = k, v
            att = np.empty(s.n_embd)
            g = s.n_head // s.n_head_kv
            for h in range(s.n_head):
                kh = h // g
                K = self.kc[l, :pos + 1, kh * d:(kh + 1) * d]
                V = self.vc[l, :pos + 1, kh * d:(kh + 1) * d]
                sc = K @ q[h * d:(h + 1) * d] / np.sqrt(d)
                pr = np.exp(sc - sc.max())
                att[h * d:(h + 1) * d] = (pr / pr.sum()) @ V
            o = w[p + "attn_output.weight"] @ att
            x = x + o if residual else o
            xb = self.rms(x, w[p + "ffn_norm.weight"], s.rms_norm_eps)
            gt = w[p + "ffn_gate.weight"] @ xb
            up = w[p + "ffn_up.weight"] @ xb
            h = gt / (1.0 + np.exp(-silu_sign * gt)) * up
            x = x + w[p + "ffn_down.weight"] @ h
        x = self.rms(x, w["output_norm.weight"], s.rms_norm_eps)
        return w["output.weight"] @ x
