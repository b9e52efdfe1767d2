"""CPU restatement of the reference decoder step ``PagedQwenDecoderStep``.

Oracle (test infrastructure only).  Restates
history/attempts/g4c-attempt69b-b4-eager/batched_decoder_step.py:197-417
("DEC" below) with the module constants (DEC:19-36) turned into parameters so
the same code serves every workload: the tiny fp32 model, one 7B layer, the
full 7B model and the B=64 scaled batch.

The op sequence and every rounding point of DEC are kept:

* RMSNorm: fp32 mean of squares, ``rsqrt(var + eps)``, cast to T, then a T x T
  product with the weight (DEC:224-229).
* q/k/v ``F.linear`` with bias, o/gate/up/down/LM-head ``x @ W.T`` in T
  (g4a_linear_t_bias.py:18-21, g4a_linear_t.py:17-18: both are plain
  ``F.linear`` / ``torch.mm`` in eager mode).
* RoPE with cos/sin computed in fp32 and cast to T, ``rotate_half``
  (DEC:231-240, 323-324).
* paged slot write (active rows only) and dense gather of the logical window
  through the block table (DEC:242-275); the caches hold post-RoPE keys.
* GQA head ``h`` reads KV head ``h // G`` (DEC:334-355).
* ExactQk: T inputs, fp32 accumulate, output rounded to bf16 (the custom op
  is bf16-out, qk-attempt50/export_qk_attempt50_air.py:51-56); scale by
  ``1/sqrt(d)`` in fp32 and round to bf16 (DEC:368); Bf16Barrier is the
  identity (bf16-barrier/export_barrier_probe.py:30-31).
* mask with the bf16 minimum where ``offset >= seq_len`` (DEC:370-374),
  softmax in fp32, probabilities rounded to bf16 (DEC:375), ``P @ V`` (DEC:376).
* o-projection, Bf16Materialize (identity), residual add in T (DEC:380-386);
  SwiGLU MLP and residual (DEC:388-403); final norm, LM head in T then
  ``.float()`` (DEC:405-408); ``next_position`` (DEC:409-411).

Decisions where DEC hard-codes values the workloads break (each recorded in
the code below):

* N1 the logical window ``window`` (DEC:33 hard-codes 8) is a parameter; the
  gather covers ``window`` logical positions of each row.
* N3 for the fp32 model the bf16 rounding points stay (scores and
  probabilities are rounded to bf16, DEC:368/375), ExactQk rounds to the
  compute dtype T instead of bf16 (it is defined on bf16 only) and the
  probabilities are cast to T before ``P @ V`` (DEC:376 would mix dtypes).

Parity pinning (tests/test_oracle_decoder.py): the whole step is checked
against HF ``Qwen2ForCausalLM`` eager (``oracle.hf_reference``, the
reference's own gate DEC:477-518) at tolerance, with weights that make the
attention scores O(1); planted mistakes (rotate_half sign, GQA head mapping,
dropped biases, RoPE base, norm weight, softmax scale) fail that gate; in
bf16 every step's logits and the K/V each layer writes equal HF eager's bit
for bit, with those weights and with the seeded N(0, 0.02) ones (HF eager
rounds at DEC's points); invariants DEC fixes exactly (masked
positions, block placement, slot-write addressing and order, inactive rows,
row independence) are checked bit for bit.  Parity unpinned: the bf16
rounding of scores and probabilities kept by the fp32 model (N3, no
independent check), and the fp32 accumulation order inside ExactQk, a closed
Ascend custom kernel (export_qk_attempt50_air.py) that cannot run here.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

BF16_MIN = torch.finfo(torch.bfloat16).min


@dataclass(frozen=True)
class ModelDims:
    """Qwen2 decoder shape (DEC:19-28 for the 7B values)."""

    num_layers: int
    hidden: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rope_theta: float = 1_000_000.0
    rms_eps: float = 1e-6
    dtype: str = "bf16"

    @property
    def torch_dtype(self) -> torch.dtype:
        return {"bf16": torch.bfloat16, "fp32": torch.float32}[self.dtype]

    @property
    def groups(self) -> int:
        return self.num_heads // self.num_kv_heads


@dataclass(frozen=True)
class PagedGeometry:
    """Paged-KV layout of one engine (DEC:29-33 for the reference B=4 values)."""

    batch: int
    physical_blocks: int
    block_size: int
    blocks_per_row: int
    window: int  # logical capacity: positions gathered per row per layer

    def __post_init__(self) -> None:
        if self.window > self.blocks_per_row * self.block_size:
            raise ValueError("logical window exceeds the blocks a row owns")


QWEN25_7B = ModelDims(
    num_layers=28,
    hidden=3584,
    num_heads=28,
    num_kv_heads=4,
    head_dim=128,
    intermediate=18944,
    vocab=152064,
)

LAYER_NAMES = (
    "input_norm",
    "post_norm",
    "q_weight",
    "q_bias",
    "k_weight",
    "k_bias",
    "v_weight",
    "v_bias",
    "o_weight",
    "gate_weight",
    "up_weight",
    "down_weight",
)


def weight_shapes(dims: ModelDims) -> dict[str, tuple[int, ...]]:
    """Tensor names and shapes of the weight bundle
    (materialize_runtime_weights.py:53-80, 83-120; DEC:43-91)."""
    kv = dims.num_kv_heads * dims.head_dim
    qd = dims.num_heads * dims.head_dim
    shapes: dict[str, tuple[int, ...]] = {"embedding": (dims.vocab, dims.hidden)}
    for layer in range(dims.num_layers):
        p = f"layers_{layer}_"
        shapes[p + "input_norm"] = (dims.hidden,)
        shapes[p + "post_norm"] = (dims.hidden,)
        shapes[p + "q_weight"] = (qd, dims.hidden)
        shapes[p + "q_bias"] = (qd,)
        shapes[p + "k_weight"] = (kv, dims.hidden)
        shapes[p + "k_bias"] = (kv,)
        shapes[p + "v_weight"] = (kv, dims.hidden)
        shapes[p + "v_bias"] = (kv,)
        shapes[p + "o_weight"] = (dims.hidden, qd)
        shapes[p + "gate_weight"] = (dims.intermediate, dims.hidden)
        shapes[p + "up_weight"] = (dims.intermediate, dims.hidden)
        shapes[p + "down_weight"] = (dims.hidden, dims.intermediate)
    shapes["final_norm"] = (dims.hidden,)
    shapes["lm_head"] = (dims.vocab, dims.hidden)
    return shapes


def rms_norm(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """DEC:224-229."""
    hidden_fp32 = hidden.float()
    variance = hidden_fp32.pow(2).mean(dim=-1, keepdim=True)
    normalized = (hidden_fp32 * torch.rsqrt(variance + eps)).to(hidden.dtype)
    return normalized * weight


def rotate_half(value: torch.Tensor) -> torch.Tensor:
    """DEC:231-233."""
    half = value.shape[-1] // 2
    return torch.cat((-value[..., half:], value[..., :half]), dim=-1)


def inv_freq(dims: ModelDims) -> torch.Tensor:
    """DEC:213-216."""
    d = dims.head_dim
    return 1.0 / (dims.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))


def rope_tables(position: torch.Tensor, dims: ModelDims, dtype: torch.dtype):
    """DEC:235-240: fp32 angles, cos/sin cast to the compute dtype."""
    batch = position.shape[0]
    freqs = position.float().reshape(batch, 1) * inv_freq(dims).view(1, dims.head_dim // 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def write_slots(
    flat: torch.Tensor,
    new_value: torch.Tensor,
    slot_mapping: torch.Tensor,
    active_mask: torch.Tensor,
) -> None:
    """Slot write of DEC:250-264, in place on ``flat`` [P*bs, KVH, d].

    DEC applies ``where(physical_slot == slot[b] & active[b], new[b], cache)``
    for b = 0..B-1 in order; a slot outside [0, P*bs) matches no physical slot
    and writes nothing; a later row overwrites an earlier one on the same
    slot.  The sequential assignment below is that, without materialising the
    full-cache ``where``.
    """
    slots = flat.shape[0]
    for b in range(new_value.shape[0]):
        s = int(slot_mapping[b])
        if int(active_mask[b]) != 0 and 0 <= s < slots:
            flat[s] = new_value[b].reshape(flat.shape[1], flat.shape[2])


def gather_window(
    flat: torch.Tensor, block_table: torch.Tensor, geometry: PagedGeometry
) -> torch.Tensor:
    """Dense gather of DEC:265-275: [B, KVH, W, d]."""
    offsets = torch.arange(geometry.window, dtype=torch.int64)
    logical_blocks = offsets // geometry.block_size
    within = offsets - logical_blocks * geometry.block_size
    physical = block_table.to(torch.int64)[:, logical_blocks]  # [B, W]
    dense_slots = physical * geometry.block_size + within  # [B, W]
    dense = flat[dense_slots.reshape(-1)].reshape(
        block_table.shape[0], geometry.window, flat.shape[1], flat.shape[2]
    )
    return dense.permute(0, 2, 1, 3).contiguous()


@dataclass
class OracleDecoder:
    """``PagedQwenDecoderStep`` over explicit weights (DEC:197-222)."""

    dims: ModelDims
    geometry: PagedGeometry
    weights: dict[str, torch.Tensor]
    _layer_cache: list = field(default_factory=list, repr=False)

    def __post_init__(self) -> None:
        shapes = weight_shapes(self.dims)
        missing = set(shapes) - set(self.weights)
        if missing:
            raise ValueError(f"missing weights: {sorted(missing)[:4]}")
        for name, shape in shapes.items():
            t = self.weights[name]
            if tuple(t.shape) != shape or t.dtype != self.dims.torch_dtype:
                raise ValueError(f"weight {name}: {tuple(t.shape)} {t.dtype}, want {shape}")

    def layer(self, index: int, name: str) -> torch.Tensor:
        return self.weights[f"layers_{index}_{name}"]

    def cache_shape(self) -> tuple[int, ...]:
        g = self.geometry
        return (
            self.dims.num_layers,
            g.physical_blocks,
            g.block_size,
            self.dims.num_kv_heads,
            self.dims.head_dim,
        )

    @torch.no_grad()
    def forward(
        self,
        token_id: torch.Tensor,
        position: torch.Tensor,
        sequence_length: torch.Tensor,
        block_table: torch.Tensor,
        slot_mapping: torch.Tensor,
        key_cache: torch.Tensor,
        value_cache: torch.Tensor,
        explicit_tiling: torch.Tensor | None,
        active_mask: torch.Tensor,
        *,
        inplace: bool = False,
    ):
        """DEC:277-417.  Inputs use the decoder ABI's Python argument order.

        Returns ``(logits fp32 [B,1,V], key_cache, value_cache, next_position)``.
        With ``inplace`` the caches are updated in place (the epoch controller
        adopts the step's output caches as its resident state, CTRL:583-584);
        otherwise they are cloned first, as DEC returns new tensors.
        """
        dims, geo = self.dims, self.geometry
        T = dims.torch_dtype
        B, H, NH, KVH, d = geo.batch, dims.hidden, dims.num_heads, dims.num_kv_heads, dims.head_dim
        G = dims.groups
        W = geo.window
        if tuple(key_cache.shape) != self.cache_shape() or key_cache.dtype != T:
            raise ValueError("key cache shape/dtype mismatch")
        if not inplace:
            key_cache = key_cache.clone()
            value_cache = value_cache.clone()

        hidden = F.embedding(token_id.reshape(B, 1).to(torch.int64), self.weights["embedding"]).view(B, 1, H)
        cos, sin = rope_tables(position.reshape(B), dims, hidden.dtype)
        cos = cos.view(B, 1, 1, d)
        sin = sin.view(B, 1, 1, d)
        valid = torch.arange(W, dtype=torch.int32).view(1, W) < sequence_length.reshape(B, 1).to(torch.int32)
        scale = math.sqrt(d)
        for li in range(dims.num_layers):
            residual = hidden
            normalized = rms_norm(hidden, self.layer(li, "input_norm"), dims.rms_eps).reshape(-1, H)
            query = F.linear(normalized, self.layer(li, "q_weight"), self.layer(li, "q_bias"))
            key = F.linear(normalized, self.layer(li, "k_weight"), self.layer(li, "k_bias"))
            value = F.linear(normalized, self.layer(li, "v_weight"), self.layer(li, "v_bias"))
            query = query.view(B, 1, NH, d).transpose(1, 2)
            key = key.view(B, 1, KVH, d).transpose(1, 2)
            value = value.view(B, 1, KVH, d).transpose(1, 2)
            query = query * cos + rotate_half(query) * sin
            key = key * cos + rotate_half(key) * sin

            flat_k = key_cache[li].view(-1, KVH, d)
            flat_v = value_cache[li].view(-1, KVH, d)
            write_slots(flat_k, key, slot_mapping, active_mask)
            write_slots(flat_v, value, slot_mapping, active_mask)
            dense_k = gather_window(flat_k, block_table, geo)  # [B, KVH, W, d]
            dense_v = gather_window(flat_v, block_table, geo)
            exp_k = dense_k.unsqueeze(2).expand(B, KVH, G, W, d).reshape(B, NH, W, d)
            exp_v = dense_v.unsqueeze(2).expand(B, KVH, G, W, d).reshape(B, NH, W, d)

            # ExactQk: T inputs, fp32 accumulation, output in bf16 (T for fp32, N3).
            qk_out = torch.bfloat16 if T == torch.bfloat16 else T
            raw_qk = torch.matmul(query.float(), exp_k.float().transpose(-1, -2)).to(qk_out)
            scores = (raw_qk.float() / scale).to(torch.bfloat16)  # DEC:368
            scores = torch.where(
                valid.view(B, 1, 1, W), scores, torch.full_like(scores, BF16_MIN)
            )  # DEC:370-374
            probabilities = torch.softmax(scores.float(), dim=-1).to(torch.bfloat16)  # DEC:375
            attention = torch.matmul(probabilities.to(T), exp_v)  # DEC:376 (N3 cast)
            attention = attention.transpose(1, 2).reshape(B, NH * d)
            projection = torch.mm(attention, self.layer(li, "o_weight").t()).reshape(B, 1, H)
            hidden = residual + projection

            residual = hidden
            normalized = rms_norm(hidden, self.layer(li, "post_norm"), dims.rms_eps).reshape(-1, H)
            gate = F.silu(torch.mm(normalized, self.layer(li, "gate_weight").t()))
            up = torch.mm(normalized, self.layer(li, "up_weight").t())
            product = gate * up
            down = torch.mm(product, self.layer(li, "down_weight").t()).reshape(B, 1, H)
            hidden = residual + down

        hidden = rms_norm(hidden, self.weights["final_norm"], dims.rms_eps)
        logits = torch.mm(hidden.reshape(-1, H), self.weights["lm_head"].t()).reshape(B, 1, dims.vocab).float()
        next_position = torch.where(active_mask.reshape(B).to(torch.bool), position.reshape(B) + 1, position.reshape(B))
        return logits, key_cache, value_cache, next_position
