"""TinyLlama-shaped CPU reference forward -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's CPU ReferenceModel
(tests/cuda/cuda_model_runner_test.cpp:213-441): fp32 arithmetic with every
activation rounded to fp16 (round to nearest even, the oracle's pinned codec)
at the same points -- matvec outputs (q, k, v, o, gate, up, down), RMSNorm
outputs, RoPE outputs, attention outputs, SwiGLU outputs and residual sums --
and fp32 logits.  Weights are the runner's seeded ones: element (r, c) of the
tensor with first row row0 is fp16(float(synth(seed, row0 + r, c)) * 0.017320508)
(N(0, 0.02) from the synthetic generator, whose std is 2/sqrt(3)); RMSNorm
weights are one.  Row ids: (layer + 1) << 40 | kind << 32, with layer ==
layer_count for the embedding and the LM head.

Only tests/ and bench.py's check may import this module.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import f16_to_f32, f32_to_f16, synth_rows

WEIGHT_SCALE = np.float32(0.017320508)
KIND = {"q": 1, "k": 2, "v": 3, "o": 4, "gate": 5, "up": 6, "down": 7, "embed": 8, "head": 9}


@dataclass(frozen=True)
class ModelConfig:
    hidden_size: int
    intermediate_size: int
    layer_count: int
    attention_head_count: int
    kv_head_count: int
    head_dimension: int
    vocabulary_size: int
    max_position_embeddings: int
    bos_token_id: int = 1
    eos_token_id: int = 2
    rms_norm_epsilon: float = 1e-5
    rope_theta: float = 10000.0


def rounded(x) -> np.ndarray:
    """fp32 -> fp16 (RNE) -> fp32 through the oracle's codec."""
    return f16_to_f32(f32_to_f16(np.asarray(x, dtype=np.float32)))


def weight_row(layer: int, kind: str) -> int:
    return ((layer + 1) << 40) | (KIND[kind] << 32)


def seeded_weight(seed: int, rows: int, cols: int, row0: int) -> np.ndarray:
    codes = synth_rows(rows * cols, seed, row0, cols)
    return rounded(f16_to_f32(codes) * WEIGHT_SCALE).reshape(rows, cols)


def matvec(w: np.ndarray, x: np.ndarray, round_output: bool = True) -> np.ndarray:
    """fp32 matrix-vector product (fp32 accumulation, like the reference's loop)."""
    y = np.dot(w, x.astype(np.float32)).astype(np.float32)
    return rounded(y) if round_output else y


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    sq = np.float32(np.sum(x.astype(np.float64) ** 2))
    scale = np.float32(1.0) / np.sqrt(sq / np.float32(x.size) + np.float32(eps), dtype=np.float32)
    return rounded(x * scale * weight)


def matmul_rows(x: np.ndarray, w: np.ndarray, round_output: bool = True) -> np.ndarray:
    """Row-wise matvec of every row of x ([n][in]) by w ([out][in]) as one fp32
    product (fp32 accumulation; the summation order may differ from
    matvec's, a difference below fp16 resolution in almost every output)."""
    y = np.dot(x.astype(np.float32), w.T).astype(np.float32)
    return rounded(y) if round_output else y


def rms_norm_rows(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """rms_norm of every row of x ([n][hidden])."""
    sq = np.sum(x.astype(np.float64) ** 2, axis=1).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(sq / np.float32(x.shape[1]) + np.float32(eps), dtype=np.float32)
    return rounded(x * scale[:, None] * weight)


def apply_rope_rows(v: np.ndarray, heads: int, dim: int, positions: np.ndarray, theta: float) -> np.ndarray:
    """apply_rope of row i of v ([n][heads * dim]) at positions[i]."""
    half = dim // 2
    n = v.shape[0]
    out = v.copy().reshape(n, heads, dim)
    d = np.arange(half, dtype=np.float32)
    inv = np.power(np.float32(theta), np.float32(-2.0) * d / np.float32(dim), dtype=np.float32)
    angle = positions.astype(np.float32)[:, None] * inv[None, :]
    c = np.cos(angle).astype(np.float32)[:, None, :]
    s = np.sin(angle).astype(np.float32)[:, None, :]
    left, right = out[:, :, :half].copy(), out[:, :, half:].copy()
    out[:, :, :half] = rounded(left * c - right * s)
    out[:, :, half:] = rounded(right * c + left * s)
    return out.reshape(n, heads * dim)


def apply_rope(v: np.ndarray, heads: int, dim: int, position: int, theta: float) -> np.ndarray:
    half = dim // 2
    out = v.copy().reshape(heads, dim)
    d = np.arange(half, dtype=np.float32)
    angle = np.float32(position) * np.power(np.float32(theta), np.float32(-2.0) * d / np.float32(dim),
                                             dtype=np.float32)
    c, s = np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)
    left, right = out[:, :half].copy(), out[:, half:].copy()
    out[:, :half] = rounded(left * c - right * s)
    out[:, half:] = rounded(right * c + left * s)
    return out.reshape(-1)


class ReferenceModel:
    """Token-at-a-time forward with its own KV history (positions in order).
    `threads` > 1 generates the weight tensors concurrently (the generator and
    codec are C calls that release the GIL; every tensor is a pure function of
    the seed and its rows, so the weights are the same)."""

    def __init__(self, cfg: ModelConfig, seed: int, threads: int = 1):
        self.cfg = cfg
        H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocabulary_size
        QD = cfg.attention_head_count * cfg.head_dimension
        KD = cfg.kv_head_count * cfg.head_dimension
        L = cfg.layer_count
        shapes = {"q": (QD, H), "k": (KD, H), "v": (KD, H), "o": (H, H), "gate": (I, H), "up": (I, H),
                  "down": (H, I)}
        jobs = [(l, kind, rows, cols) for l in range(L) for kind, (rows, cols) in shapes.items()]
        jobs += [(L, "embed", V, H), (L, "head", V, H)]

        def make(job):
            l, kind, rows, cols = job
            return seeded_weight(seed, rows, cols, weight_row(l, kind))

        if threads > 1:
            from concurrent.futures import ThreadPoolExecutor
            with ThreadPoolExecutor(max_workers=threads) as pool:
                made = list(pool.map(make, jobs))
        else:
            made = [make(j) for j in jobs]
        tensors = {(j[0], j[1]): w for j, w in zip(jobs, made)}
        self.layers = []
        for l in range(L):
            layer = {kind: tensors[(l, kind)] for kind in shapes}
            layer["ln1"] = np.ones(H, dtype=np.float32)
            layer["ln2"] = np.ones(H, dtype=np.float32)
            self.layers.append(layer)
        self.embed = tensors[(L, "embed")]
        self.head = tensors[(L, "head")]
        self.final_norm = np.ones(H, dtype=np.float32)
        self.keys = [[] for _ in range(L)]
        self.values = [[] for _ in range(L)]
        self.final_hidden = None

    def fresh(self) -> "ReferenceModel":
        """Another request on the same weights: shares them, empty KV history."""
        other = object.__new__(ReferenceModel)
        other.__dict__.update(self.__dict__)
        L = self.cfg.layer_count
        other.keys = [[] for _ in range(L)]
        other.values = [[] for _ in range(L)]
        other.final_hidden = None
        return other

    def forward(self, token: int, position: int) -> np.ndarray:
        cfg = self.cfg
        D, QH, KVH = cfg.head_dimension, cfg.attention_head_count, cfg.kv_head_count
        G = QH // KVH
        scale = np.float32(1.0) / np.sqrt(np.float32(D))
        hidden = self.embed[token].copy()
        for l, W in enumerate(self.layers):
            x = rms_norm(hidden, W["ln1"], cfg.rms_norm_epsilon)
            q = apply_rope(matvec(W["q"], x), QH, D, position, cfg.rope_theta)
            k = apply_rope(matvec(W["k"], x), KVH, D, position, cfg.rope_theta)
            v = matvec(W["v"], x)
            self.keys[l].append(k)
            self.values[l].append(v)
            K = np.stack(self.keys[l]).reshape(-1, KVH, D).astype(np.float64)
            Vv = np.stack(self.values[l]).reshape(-1, KVH, D).astype(np.float64)
            attn = np.zeros(QH * D, dtype=np.float32)
            for h in range(QH):
                s = (K[:, h // G, :] @ q[h * D:(h + 1) * D].astype(np.float64)).astype(np.float32) * scale
                p = np.exp((s - s.max()).astype(np.float64))
                attn[h * D:(h + 1) * D] = rounded(((p / p.sum()) @ Vv[:, h // G, :]).astype(np.float32))
            hidden = rounded(hidden + matvec(W["o"], attn))
            x = rms_norm(hidden, W["ln2"], cfg.rms_norm_epsilon)
            gate, up = matvec(W["gate"], x), matvec(W["up"], x)
            act = rounded(gate / (np.float32(1.0) + np.exp(-gate)) * up)
            hidden = rounded(hidden + matvec(W["down"], act))
        self.final_hidden = rms_norm(hidden, self.final_norm, cfg.rms_norm_epsilon)
        return matvec(self.head, self.final_hidden, round_output=False)

    @staticmethod
    def _span_mask(positions: np.ndarray, total: int) -> np.ndarray:
        """Causal mask of the span's rows (at `positions`) over the history +
        span keys [0, total)."""
        return np.arange(total)[None, :] <= positions[:, None]

    def forward_span(self, tokens, first_position: int) -> np.ndarray:
        """The token-at-a-time forward of tokens at positions first_position,
        first_position + 1, ... (the next positions of this request), with the
        span's rows batched into matrix products and its causal attention
        computed for all rows at once; same fp16 rounding points and the same
        KV history afterwards.  Returns the logits after the span's last
        token.  Agrees with forward() token by token within fp16 noise (only
        the fp32 summation order of the products differs)."""
        cfg = self.cfg
        D, QH, KVH = cfg.head_dimension, cfg.attention_head_count, cfg.kv_head_count
        G = QH // KVH
        n = len(tokens)
        assert n > 0 and len(self.keys[0]) == first_position
        positions = np.arange(first_position, first_position + n)
        scale = np.float32(1.0) / np.sqrt(np.float32(D))
        hidden = self.embed[np.asarray(tokens, dtype=np.int64)].copy()
        total = first_position + n
        allowed = self._span_mask(positions, total)
        for l, W in enumerate(self.layers):
            x = rms_norm_rows(hidden, W["ln1"], cfg.rms_norm_epsilon)
            q = apply_rope_rows(matmul_rows(x, W["q"]), QH, D, positions, cfg.rope_theta)
            k = apply_rope_rows(matmul_rows(x, W["k"]), KVH, D, positions, cfg.rope_theta)
            v = matmul_rows(x, W["v"])
            self.keys[l].extend(list(k))
            self.values[l].extend(list(v))
            K = np.stack(self.keys[l]).reshape(total, KVH, D).astype(np.float64)
            Vv = np.stack(self.values[l]).reshape(total, KVH, D).astype(np.float64)
            attn = np.zeros((n, QH * D), dtype=np.float32)
            q64 = q.reshape(n, QH, D).astype(np.float64)
            for h in range(QH):
                s = (q64[:, h, :] @ K[:, h // G, :].T).astype(np.float32) * scale        # [n][total]
                s = np.where(allowed, s, np.float32(-np.inf))
                p = np.exp((s - s.max(axis=1, keepdims=True)).astype(np.float64))
                attn[:, h * D:(h + 1) * D] = rounded(((p / p.sum(axis=1, keepdims=True)) @ Vv[:, h // G, :])
                                                     .astype(np.float32))
            hidden = rounded(hidden + matmul_rows(attn, W["o"]))
            x = rms_norm_rows(hidden, W["ln2"], cfg.rms_norm_epsilon)
            gate, up = matmul_rows(x, W["gate"]), matmul_rows(x, W["up"])
            act = rounded(gate / (np.float32(1.0) + np.exp(-gate)) * up)
            hidden = rounded(hidden + matmul_rows(act, W["down"]))
        self.final_hidden = rms_norm(hidden[-1], self.final_norm, cfg.rms_norm_epsilon)
        return matvec(self.head, self.final_hidden, round_output=False)

    def generate(self, prompt, max_new_tokens: int, eos: int | None = None):
        """Greedy generation (tests/cuda/cuda_model_runner_test.cpp:423-443)."""
        logits = None
        for p, t in enumerate(prompt):
            logits = self.forward(int(t), p)
        out = []
        for g in range(max_new_tokens):
            nxt = int(np.argmax(logits))
            out.append(nxt)
            if (eos is not None and nxt == eos) or g + 1 == max_new_tokens:
                break
            logits = self.forward(nxt, len(prompt) + g)
        return out
