"""One decode token on the device: the projection sequence of DenseForward.Step and Final
(src/Satori.Core/Model/DenseForward.cs:100-162, 298-306) over resident quantized matrices, with the operators
of TransformerOps (src/Satori.Core/TransformerOps.cs) between the projections, the key/value cache on the
device, and the whole token recordable as one replayable step (HipContext.capture_begin / capture_end).

Per layer: RmsNorm -> q/k/v projections (one group launch) -> bias adds (k and v written straight into the
cache slot) -> half-split RoPE of q and the new key -> grouped attention over the cached prefix -> o projection
-> residual add -> RmsNorm -> gate/up projections (one group launch) -> SwiGLU -> down projection -> residual
add. Then the final RmsNorm and the output projection. The K-format projections quantize their input to Q8_K
inside their own launch, so no separate quantization runs. By default the attention inputs (bias adds, RoPE,
cache writes) are one launch and each residual add shares a launch with the RmsNorm after it: 9 launches per
layer instead of 14, with bit-identical results. Folded (`folded=True`), the residual add + RmsNorm before
q/k/v and before gate/up is computed inside those projection launches (group input transforms; the residual
alternates between two buffers, since the launch that writes it is also read by its other workgroups), the
attention inputs run inside the split attention, and the add + RmsNorm before the output projection, whose
launch has 2,374 workgroups, is one single-workgroup launch that also writes the Q8_K bytes the projection
reads (computed in each of its workgroups it costs more than the launch; for gate/up, with 560 workgroups,
the fold measured faster). SwiGlu is carried by the gate/up launch itself (its workgroups own the same rows
of gate and up), and the down projection quantizes that vector in its own launch (folded into down instead,
every down workgroup would evaluate the FP64 exponentials of the whole 8960-wide vector: measured 2.12 ms per
token that way). Again bit-identical results.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import DeviceOps, HipContext, HipGroup, HipQuantizedMatrix, HipStep


def decode_attention_launches(tokens: int, head_dim: int) -> int:
    """Launches of satori_hip_attention_decode over `tokens` cached tokens, by the library's rule: up to 32
    tokens, the attention inputs and the one-workgroup attention (2); beyond, the split attention over
    max(min(32, ceil(tokens / 32)), min(64, ceil(tokens / 128)), ceil(tokens / 2048)) workgroups per head,
    with the inputs inside it (split + combine: 2) while the head fits one workgroup's lanes (at most 256)
    and each split holds at most 80 tokens, else beside it (inputs + split + combine: 3)."""
    if tokens <= 32:
        return 2
    splits = max(min(32, (tokens + 31) // 32), min(64, (tokens + 127) // 128), (tokens + 2047) // 2048)
    per = -(-tokens // splits)
    fits = per * 8 + 3 * head_dim * 4 + 256 * 8 <= 64 * 1024
    return 2 if head_dim <= 256 and per <= 80 and fits else 3


@dataclass
class DecoderConfig:
    hidden: int          # embedding width
    heads: int           # query heads
    kv_heads: int        # key/value heads
    head_dim: int
    ffn: int             # feed-forward width
    epsilon: float       # RMS norm epsilon
    rope_base: float     # RoPE frequency base
    max_tokens: int      # key/value cache capacity (positions)


class DeviceDecoder:
    """Resident decode loop. `layers[i]` maps "q", "k", "v", "o", "gate", "up", "down" to resident matrices;
    `vectors[i]` maps "attn_norm", "ffn_norm" (and optionally "q_bias", "k_bias", "v_bias") to device
    pointers of FP32 vectors; `output_norm` is a device pointer, `output` the output projection and
    `embedding` the token-embedding matrix (its rows are decoded on the device, GgufQuantizedMatrix.ReadRow)."""

    def __init__(self, context: HipContext, config: DecoderConfig, layers: list[dict], vectors: list[dict],
                 output_norm: int, output: HipQuantizedMatrix, embedding: HipQuantizedMatrix):
        self.ctx, self.cfg = context, config
        self.layers, self.vectors = layers, vectors
        self.output_norm, self.output, self.embedding = output_norm, output, embedding
        self.ops = DeviceOps(context)
        c = config
        self.q_width = c.heads * c.head_dim
        self.kv_width = c.kv_heads * c.head_dim
        self._buffers = []
        self.groups = []
        self.final = None
        self._folded = None  # groups with input transforms, made on first use
        try:
            self._build(context, config, layers, output)
        except BaseException:
            self.dispose()  # nothing half-built stays allocated or holds the caller's matrices
            raise

    def _build(self, context: HipContext, c: DecoderConfig, layers: list[dict], output: HipQuantizedMatrix) -> None:
        def buf(n):
            p = context.alloc(4 * n)
            self._buffers.append(p)
            context.upload(p, np.zeros(n, np.float32))
            return p

        self.residual, self.normed = buf(c.hidden), buf(c.hidden)
        self.residual_b = buf(c.hidden)  # the folded sequence's second residual buffer
        self.q, self.k, self.v = buf(self.q_width), buf(self.kv_width), buf(self.kv_width)
        self.context_vec, self.projected = buf(self.q_width), buf(c.hidden)
        self.gate, self.up, self.activated = buf(c.ffn), buf(c.ffn), buf(c.ffn)
        self.logits = buf(output.rows)
        self.activated_q8k = buf(c.ffn // 256 * 73)  # Q8_K bytes of the down projection's input (292 per block)
        self.normed_q8k = buf(c.hidden // 256 * 73)  # Q8_K bytes of the output projection's input
        self.zero_kv = buf(self.kv_width)
        self.keys = [buf(c.max_tokens * self.kv_width) for _ in layers]
        self.values = [buf(c.max_tokens * self.kv_width) for _ in layers]
        # RoPE sines and cosines of every cache position (doubles), computed once for the session.
        self.rope = buf(2 * c.max_tokens * c.head_dim)
        self.ops.rope_table(c.max_tokens, c.head_dim, c.rope_base, self.rope)
        for m in layers:
            group = {}
            self.groups.append(group)
            group["qkv"] = HipGroup(context, [m["q"], m["k"], m["v"]], [self.normed] * 3, [self.q, self.k, self.v],
                                    True)
            group["o"] = HipGroup(context, [m["o"]], [self.context_vec], [self.projected], True)
            group["gateup"] = HipGroup(context, [m["gate"], m["up"]], [self.normed] * 2, [self.gate, self.up], True)
            group["down"] = HipGroup(context, [m["down"]], [self.activated], [self.projected], True)
        self.final = HipGroup(context, [output], [self.normed], [self.logits], True)
        # The split attention's workspace is allocated by its first call and covers every shorter prefix of
        # these heads: make that call now at the cache capacity, so that a token can be captured before any
        # has run.
        self.ops.grouped_attention(self.q, self.keys[0], self.values[0], c.heads, c.kv_heads, c.head_dim,
                                   c.max_tokens, self.context_vec)

    def _folded_groups(self):
        """Per layer the q/k/v group reading RmsNorm(residual + previous down output) (layer 0: RmsNorm of the
        embedding row) and writing the sum to the second residual buffer, the gate/up group reading
        RmsNorm(second residual + o output), writing the sum back and carrying SwiGlu, and the down group
        reading that vector; then the output group reading the Q8_K bytes of RmsNorm(residual + last down
        output)."""
        if self._folded is None:
            c, ctx = self.cfg, self.ctx
            folded = []
            for layer, (m, vec) in enumerate(zip(self.layers, self.vectors)):
                read, written = self.residual, self.residual_b
                qkv = HipGroup(ctx, [m["q"], m["k"], m["v"]], [self.normed] * 3, [self.q, self.k, self.v], True)
                qkv.set_input_add_rms_norm(read, self.projected if layer else 0, vec["attn_norm"], c.epsilon, written)
                gateup = HipGroup(ctx, [m["gate"], m["up"]], [self.normed] * 2, [self.gate, self.up], True)
                gateup.set_input_add_rms_norm(written, self.projected, vec["ffn_norm"], c.epsilon, read)
                gateup.set_output_swiglu(self.activated)
                down = HipGroup(ctx, [m["down"]], [self.activated], [self.projected], True)
                folded.append({"qkv": qkv, "gateup": gateup, "down": down})
            final = HipGroup(ctx, [self.output], [self.normed], [self.logits], True)
            final.set_input_q8k(self.normed_q8k)
            self._folded = (folded, final)
        return self._folded

    def enqueue(self, token: int, position: int, fused: bool = True, folded: bool = False) -> None:
        """Enqueues one token at `position` (keys/values of positions < position are in the cache). Fused:
        the bias adds, RoPE and cache writes of a layer's attention inputs are one launch, and every residual
        add shares its launch with the RmsNorm that follows (bit-identical to the unfused sequence). Folded:
        as fused, with the residual adds and RmsNorms computed inside the projections that consume them and the
        attention inputs inside the split attention (bit-identical as well)."""
        c, ops = self.cfg, self.ops
        if not 0 <= position < c.max_tokens:
            raise ValueError("position outside the key/value cache")
        self.embedding.decode_row_device(token, self.residual)
        if folded:
            groups, final = self._folded_groups()
            for layer, (g, fg, vec) in enumerate(zip(self.groups, groups, self.vectors)):
                fg["qkv"].execute()
                ops.attention_decode(self.q, vec.get("q_bias", 0), self.k, vec.get("k_bias", 0), self.v,
                                     vec.get("v_bias", 0), self.keys[layer], self.values[layer], c.heads, c.kv_heads,
                                     c.head_dim, position, c.rope_base, c.head_dim, self.context_vec, self.rope)
                g["o"].execute()
                fg["gateup"].execute()  # also SwiGlu
                fg["down"].execute()
            ops.add_rms_norm_q8k(self.residual, self.projected, self.output_norm, c.epsilon, c.hidden, self.normed,
                                 self.normed_q8k)
            final.execute()
            return
        if fused:
            ops.rms_norm(self.residual, self.vectors[0]["attn_norm"], c.epsilon, c.hidden, self.normed)
        for layer, (g, vec) in enumerate(zip(self.groups, self.vectors)):
            k_slot = self.keys[layer] + 4 * position * self.kv_width
            v_slot = self.values[layer] + 4 * position * self.kv_width
            if not fused:
                ops.rms_norm(self.residual, vec["attn_norm"], c.epsilon, c.hidden, self.normed)
            g["qkv"].execute()
            if fused:
                ops.attention_inputs(self.q, vec.get("q_bias", 0), self.k, vec.get("k_bias", 0), k_slot, self.v,
                                     vec.get("v_bias", 0), v_slot, c.heads, c.kv_heads, c.head_dim, position,
                                     c.rope_base, c.head_dim)
            else:
                if "q_bias" in vec:
                    ops.add(self.q, vec["q_bias"], self.q_width, self.q)
                ops.add(self.k, vec.get("k_bias", self.zero_kv), self.kv_width, k_slot)
                ops.add(self.v, vec.get("v_bias", self.zero_kv), self.kv_width, v_slot)
                ops.rope_half(self.q, self.q_width, c.head_dim, position, c.rope_base, c.head_dim)
                ops.rope_half(k_slot, self.kv_width, c.head_dim, position, c.rope_base, c.head_dim)
            ops.grouped_attention(self.q, self.keys[layer], self.values[layer], c.heads, c.kv_heads, c.head_dim,
                                  position + 1, self.context_vec)
            g["o"].execute()
            if fused:
                ops.add_rms_norm(self.residual, self.projected, vec["ffn_norm"], c.epsilon, c.hidden, self.normed)
            else:
                ops.add(self.residual, self.projected, c.hidden, self.residual)
                ops.rms_norm(self.residual, vec["ffn_norm"], c.epsilon, c.hidden, self.normed)
            g["gateup"].execute()
            ops.swiglu(self.gate, self.up, c.ffn, self.activated)
            g["down"].execute()
            if fused:
                following = (self.vectors[layer + 1]["attn_norm"] if layer + 1 < len(self.groups)
                             else self.output_norm)
                ops.add_rms_norm(self.residual, self.projected, following, c.epsilon, c.hidden, self.normed)
            else:
                ops.add(self.residual, self.projected, c.hidden, self.residual)
        if not fused:
            ops.rms_norm(self.residual, self.output_norm, c.epsilon, c.hidden, self.normed)
        self.final.execute()

    def launches_per_token(self, fused: bool = True, folded: bool = False, position: int | None = None) -> int:
        """Kernel launches of one token. At a `position` whose prefix exceeds 32 tokens the attention is split
        over several workgroups per head and combined by a second kernel, one more launch per layer."""
        split = position is not None and position + 1 > 32
        extra = len(self.layers) if split else 0
        if folded:  # q/k/v, the decode attention, o, gate/up (and SwiGlu), down; add + RmsNorm to Q8_K, output
            attention = decode_attention_launches(position + 1 if position is not None else 1, self.cfg.head_dim)
            return 1 + (4 + attention) * len(self.layers) + 2
        if fused:
            return 2 + 9 * len(self.layers) + 1 + extra
        per_layer = 14 if all("q_bias" in v for v in self.vectors) else 13
        return 1 + per_layer * len(self.layers) + 2 + extra

    def capture(self, token: int, position: int, fused: bool = True, folded: bool = False) -> HipStep:
        """The token at `position` recorded as one replayable step."""
        if folded:
            self._folded_groups()  # created (and their transforms set) before capturing
        self.ctx.capture_begin()
        try:
            self.enqueue(token, position, fused, folded)
        except BaseException:
            self.ctx.capture_end().dispose()
            raise
        return self.ctx.capture_end()

    def read_logits(self) -> np.ndarray:
        out = np.zeros(self.output.rows, np.float32)
        self.ctx.synchronize()
        return self.ctx.download(out, self.logits)

    def dispose(self) -> None:
        for g in self.groups:
            for gr in g.values():
                gr.dispose()
        self.groups = []
        if self.final is not None:
            self.final.dispose()
            self.final = None
        if self._folded is not None:
            for g in self._folded[0]:
                for gr in g.values():
                    gr.dispose()
            self._folded[1].dispose()
            self._folded = None
        for p in self._buffers:
            self.ctx.free(p)
        self._buffers = []
