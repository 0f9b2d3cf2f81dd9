"""Pins the oracle's decoder step (orc_decoder_*) against an independent FP64 numpy decoder written from the
reference's step description (step.rs:137-185, step/layers.rs:31-228, elementwise.cu:3-109): exact dequantized
weights, FP64 arithmetic, NeoX RoPE from the same tables, causal attention over each slot's positions. A dropped
residual, a transposed projection, a wrong norm or a rotated V fails by far more than the FP32 rounding of the
oracle (bar: 1e-4 x the logits range). Closed forms pin the RMS norm and SwiGLU pieces on their own.
"""

import numpy as np
import pytest

from oracle_ffi import DecoderOracle
from synapse_amd.decoder import LAYER_MATRICES, DecoderShape, q4_k_m, synthetic_model
from synapse_amd.projection import dequantize, dequantize_q8_0, matrix_bytes

TINY = DecoderShape(layers=2, hidden=128, feed_forward=256, heads=2, kv_heads=1, head_dim=64, vocabulary=96,
                    context=256, session_slots=3, step_tokens=16, logits_rows=8, growth=64)


def rope_tables(head_dim, theta, positions):
    """RopeFrequencies (RopeFrequencies.cs:55-81) restated in numpy: FP32 tables of cos/sin(p * theta^(-2i/d))."""
    half = head_dim // 2
    inverse = (np.float64(theta) ** (-np.arange(half, dtype=np.float64) * 2.0 / head_dim))
    angles = np.arange(positions, dtype=np.float64)[:, None] * inverse[None, :]
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


class NumpyDecoder:
    """FP64 decoder over exactly dequantized weights (the independent check)."""

    def __init__(self, blob, layout, shape, cosines, sines):
        s = shape
        self.s = s
        self.cos = cosines.astype(np.float64)
        self.sin = sines.astype(np.float64)

        def matrix(offset, rows, columns, encoding=8):
            size = matrix_bytes(encoding, rows, columns)
            return dequantize(encoding, blob[offset:offset + size], columns).astype(np.float64)

        def vector(offset, count):
            if offset == (1 << 64) - 1:
                return np.zeros(count)
            return blob[offset:offset + 4 * count].view(np.float32).astype(np.float64)

        kv = s.kv_width
        self.embedding = matrix(layout["token_embedding"], s.vocabulary, s.hidden, layout.get("embedding_encoding", 8))
        self.output = matrix(layout["output"], s.vocabulary, s.hidden, layout.get("output_encoding", 8))
        self.output_norm = vector(layout["output_norm"], s.hidden)
        self.layers = []
        for layer in layout["layers"]:
            enc = {name: (int(layer["encodings"]) >> (4 * index)) & 0xF for index, name in enumerate(LAYER_MATRICES)}
            self.layers.append({
                "attention_norm": vector(layer["attention_norm"], s.hidden),
                "q": matrix(layer["query"], s.hidden, s.hidden, enc["attn_q"]),
                "qb": vector(layer["query_bias"], s.hidden),
                "k": matrix(layer["key"], kv, s.hidden, enc["attn_k"]), "kb": vector(layer["key_bias"], kv),
                "v": matrix(layer["value"], kv, s.hidden, enc["attn_v"]), "vb": vector(layer["value_bias"], kv),
                "o": matrix(layer["attention_output"], s.hidden, s.hidden, enc["attn_output"]),
                "ffn_norm": vector(layer["feed_forward_norm"], s.hidden),
                "gate": matrix(layer["gate"], s.feed_forward, s.hidden, enc["ffn_gate"]),
                "up": matrix(layer["up"], s.feed_forward, s.hidden, enc["ffn_up"]),
                "down": matrix(layer["down"], s.hidden, s.feed_forward, enc["ffn_down"]),
            })
        self.keys = {}    # (slot, layer) -> {position: [kv_heads, head_dim]}
        self.values = {}

    def norm(self, x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.s.rms_epsilon) * w

    def rotate(self, x, position):
        half = self.s.head_dim // 2
        c, s = self.cos[position], self.sin[position]
        first, second = x[..., :half], x[..., half:]
        return np.concatenate([first * c - second * s, first * s + second * c], axis=-1)

    def forward(self, tokens):
        s = self.s
        d = s.head_dim
        group = s.heads // s.kv_heads
        hidden = np.stack([self.embedding[token] for _, token, _, _ in tokens])
        for index, layer in enumerate(self.layers):
            n = self.norm(hidden, layer["attention_norm"])
            q = (n @ layer["q"].T + layer["qb"]).reshape(len(tokens), s.heads, d)
            k = (n @ layer["k"].T + layer["kb"]).reshape(len(tokens), s.kv_heads, d)
            v = (n @ layer["v"].T + layer["vb"]).reshape(len(tokens), s.kv_heads, d)
            for t, (slot, _, position, _) in enumerate(tokens):
                q[t] = self.rotate(q[t], position)
                k[t] = self.rotate(k[t], position)
                self.keys.setdefault((slot, index), {})[position] = k[t].copy()
                self.values.setdefault((slot, index), {})[position] = v[t].copy()
            attention = np.zeros((len(tokens), s.heads, d))
            for t, (slot, _, position, _) in enumerate(tokens):
                keys = np.stack([self.keys[(slot, index)][p] for p in range(position + 1)])
                values = np.stack([self.values[(slot, index)][p] for p in range(position + 1)])
                for head in range(s.heads):
                    scores = keys[:, head // group] @ q[t, head] / np.sqrt(d)
                    weights = np.exp(scores - scores.max())
                    attention[t, head] = weights @ values[:, head // group] / weights.sum()
            hidden = hidden + attention.reshape(len(tokens), -1) @ layer["o"].T
            n = self.norm(hidden, layer["ffn_norm"])
            gate = n @ layer["gate"].T
            up = n @ layer["up"].T
            hidden = hidden + (gate / (1 + np.exp(-gate)) * up) @ layer["down"].T
        rows = [t for t, token in enumerate(tokens) if token[3] >= 0]
        return self.norm(hidden[rows], self.output_norm) @ self.output.T


def steps_for(rng, shape):
    """Prompt runs, ragged decode, a token without logits and a logits row for every other token."""
    vocab = shape.vocabulary
    a = [(0, int(rng.integers(vocab)), p, -1) for p in range(10)] + [(1, int(rng.integers(vocab)), p, -1)
                                                                       for p in range(5)]
    a = [(slot, token, position, -1) for slot, token, position, _ in a]
    a[9] = a[9][:3] + (0,)
    a[14] = a[14][:3] + (1,)
    b = [(0, 7, 10, 0), (1, 8, 5, 1), (2, 9, 0, 2)]
    c = [(2, 3, 1, -1), (0, 11, 11, 0), (1, 12, 6, 1), (2, 13, 2, 2)]
    return [a, b, c]


# K-quant matrices need whole 256-value super-blocks: hidden and feed-forward widths of 256 and 512.
TINY_K = DecoderShape(layers=2, hidden=256, feed_forward=512, heads=4, kv_heads=1, head_dim=64, vocabulary=96,
                      context=256, session_slots=3, step_tokens=16, logits_rows=8, growth=64)


@pytest.mark.parametrize("biases,encodings", [(True, None), (False, None), (True, "q4_k_m"), (False, "q6_k")])
def test_oracle_decoder_matches_fp64_numpy(biases, encodings):
    """Q8_0 models and K-quant ones (the Q4_K_M mix: Q4_K with Q6_K for V, down and output; and all Q6_K)."""
    rng = np.random.default_rng(3 + biases)
    shape = TINY if encodings is None else TINY_K
    choose = {None: None, "q4_k_m": q4_k_m, "q6_k": lambda name: 14}[encodings]
    blob, layout = synthetic_model(shape, seed=7 + biases, biases=biases, encodings=choose)
    cos, sin = rope_tables(shape.head_dim, shape.theta, shape.context)
    oracle = DecoderOracle(blob, layout, shape, cos, sin)
    reference = NumpyDecoder(blob, layout, shape, cos, sin)
    for step in steps_for(rng, shape):
        got = oracle.forward(step)
        expected = reference.forward(step)
        assert got.shape == expected.shape
        bar = 1e-4 * (expected.max() - expected.min())
        assert np.abs(got - expected).max() <= bar, (np.abs(got - expected).max(), bar)


def test_oracle_decoder_is_sensitive_to_each_piece():
    """The bar is tight enough to see one wrong piece: dropping a layer's feed-forward residual (zeroing the down
    matrix) moves the logits by far more than the bar."""
    blob, layout = synthetic_model(TINY, seed=9)
    cos, sin = rope_tables(TINY.head_dim, TINY.theta, TINY.context)
    tokens = [(0, 5, p, 0 if p == 5 else -1) for p in range(6)]
    baseline = DecoderOracle(blob, layout, TINY, cos, sin).forward(tokens)
    changed = blob.copy()
    down = layout["layers"][1]["down"]
    size = TINY.hidden * (TINY.feed_forward // 32) * 34
    changed[down:down + size] = 0
    other = DecoderOracle(changed, layout, TINY, cos, sin).forward(tokens)
    assert np.abs(other - baseline).max() > 100 * 1e-4 * (baseline.max() - baseline.min())


def test_rms_norm_and_swiglu_closed_forms():
    """A model with zero layer matrices and no biases passes the embedding row through the layers unchanged, so the
    logits are W_out (x / sqrt(mean(x^2) + eps) * w_out): computed here from the row alone."""
    shape = DecoderShape(layers=1, hidden=64, feed_forward=64, heads=1, kv_heads=1, head_dim=64, vocabulary=40,
                         context=64, session_slots=1, step_tokens=4, logits_rows=4, growth=64)
    blob, layout = synthetic_model(shape, seed=2, biases=False)
    layer = layout["layers"][0]
    for name, rows, columns in (("query", 64, 64), ("key", 64, 64), ("value", 64, 64), ("attention_output", 64, 64),
                                ("gate", 64, 64), ("up", 64, 64), ("down", 64, 64)):
        blob[layer[name]:layer[name] + rows * (columns // 32) * 34] = 0
    cos, sin = rope_tables(64, shape.theta, 64)
    logits = DecoderOracle(blob, layout, shape, cos, sin).forward([(0, 17, 0, 0), (0, 3, 1, 1)])
    embedding = dequantize_q8_0(blob[layout["token_embedding"]:layout["token_embedding"] + 40 * 2 * 34], 64)
    output = dequantize_q8_0(blob[layout["output"]:layout["output"] + 40 * 2 * 34], 64).astype(np.float64)
    w = blob[layout["output_norm"]:layout["output_norm"] + 256].view(np.float32).astype(np.float64)
    for row, token in enumerate((17, 3)):
        x = embedding[token].astype(np.float64)
        expected = output @ (x / np.sqrt(np.mean(x * x) + shape.rms_epsilon) * w)
        assert np.allclose(logits[row], expected, rtol=1e-5, atol=1e-5 * np.abs(expected).max())


def test_logits_rows_follow_token_order():
    """Only tokens with a logits row produce logits, in token order; the same token with and without a row leaves
    the other rows unchanged (per-token independence of the step)."""
    blob, layout = synthetic_model(TINY, seed=4)
    cos, sin = rope_tables(TINY.head_dim, TINY.theta, TINY.context)
    first = DecoderOracle(blob, layout, TINY, cos, sin).forward([(0, 1, 0, 0), (1, 2, 0, -1), (2, 3, 0, 1)])
    second = DecoderOracle(blob, layout, TINY, cos, sin).forward([(0, 1, 0, 0), (1, 2, 0, 1), (2, 3, 0, 2)])
    assert first.shape == (2, TINY.vocabulary)
    assert np.array_equal(first[0], second[0]) and np.array_equal(first[1], second[2])
