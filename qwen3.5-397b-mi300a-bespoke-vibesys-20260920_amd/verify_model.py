"""Compact Qwen3.5-MoE target model for the MTP verify path.

What the speculative step needs of the target, and nothing else: token embedding, a stack of
Gated-DeltaNet and gated GQA attention layers each followed by the routed MXFP4 MoE plus the
shared expert, the final norm and the LM head; a paged KV cache with 16-row blocks; per-slot
DeltaNet conv/recurrent state; and the cached last hidden state the MTP head is seeded from.
The layer math follows the reference's `Model` (`model.py:587-649` norms/RoPE/SwiGLU,
`model.py:2158-2290` gated attention, `model.py:2396-2470` DeltaNet, `model.py:2758-2873`
MoE) and its wide verify forward (`decode_layer_verify`, `model.py:3974-3995`).

Verify and commit are split differently from the reference. `deltanet_verify` computes all
`t` rows' outputs from the committed state WITHOUT writing any state back, and returns the
per-row activations; `deltanet_commit` then advances the stored conv window and recurrent
state by exactly `lengths[j]` rows of slot j. The reference writes the speculative state for
all `t` rows, snapshots the pre-verify state and replays the accepted prefix over it
(`deltanet_verify` / `deltanet_verify_rollback`, `model.py:3738-3972`); the result is the
same state, without the `[B, heads, k_dim, v_dim]` clone and its HBM round trip. Plain decode
is the same pair at `t = 1`, so a speculative round and a sequence of decode steps run the
same per-row arithmetic.

Device tensors take the HIP kernels for the routed MoE (`mxfp4_gemv.fused_moe`), the router
(`router_fused.route`) and the argmax (`mtp.argmax_rows`), and raise if the library is
missing. CPU tensors take the reference's torch spellings of the same ops (its CPU engine:
`mxfp4_gemv.reference_moe`, softmax/topk, `argmax`), which is what config 1 exercises.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

import attention
import blas_tune
import deltanet
import dense
import mxfp4
import mtp_dense_moe
import mxfp4_gemv
import router_fused
import rownorm

ATTN = "full_attention"
DELTANET = "linear_attention"


@dataclass(frozen=True)
class Cfg:
    """Model shape (the fields of the reference's `Cfg`, `model.py:530-551`, plus the expert
    intermediate width and the KV block size)."""

    hidden: int
    vocab: int
    layer_types: tuple[str, ...]
    eps: float
    heads: int
    kv_heads: int
    head_dim: int
    rot_dim: int
    rope_theta: float
    k_heads: int
    v_heads: int
    k_dim: int
    v_dim: int
    conv_k: int
    experts: int
    top_k: int
    inter: int
    shared_inter: int
    block_size: int = 16
    eos: tuple[int, ...] = ()

    @property
    def conv_dim(self) -> int:
        return 2 * self.k_heads * self.k_dim + self.v_heads * self.v_dim

    @property
    def in_proj_sizes(self) -> list[int]:
        """Output widths of the fused DeltaNet input projection: qkv, z, beta, a
        (`model.py:860-867`)."""
        return [self.conv_dim, self.v_heads * self.v_dim, self.v_heads, self.v_heads]


def tiny_cfg() -> Cfg:
    """The CPU plumbing model: hidden 64, 3 DeltaNet + 1 attention layer (4 q / 2 kv heads of
    16), 8 experts top-2 with intermediate 32, one shared expert, vocab 512."""
    return Cfg(
        hidden=64, vocab=512, layer_types=(DELTANET, DELTANET, DELTANET, ATTN), eps=1e-6,
        heads=4, kv_heads=2, head_dim=16, rot_dim=4, rope_theta=10000.0,
        k_heads=2, v_heads=4, k_dim=16, v_dim=16, conv_k=4,
        experts=8, top_k=2, inter=32, shared_inter=32, eos=(1,),
    )  # fmt: skip


def verify_cfg() -> Cfg:
    """Real Qwen3.5-397B-A17B layer dimensions at reduced depth: 3 DeltaNet + 1 gated GQA
    attention layer (32 q / 2 kv heads of 256, RoPE on the first 64 channels), 512 experts
    top-10 of intermediate 1024 plus a shared expert of 1024, vocab 248320."""
    return Cfg(
        hidden=4096, vocab=248320, layer_types=(DELTANET, DELTANET, DELTANET, ATTN), eps=1e-6,
        heads=32, kv_heads=2, head_dim=256, rot_dim=64, rope_theta=1.0e7,
        k_heads=16, v_heads=64, k_dim=128, v_dim=128, conv_k=4,
        experts=512, top_k=10, inter=1024, shared_inter=1024,
    )  # fmt: skip


# ---------------------------------------------------------------- layer math

SMALL_WEIGHT_BYTES = 32 << 20
"""Linears of at most this many weight bytes and <= 64 rows take the skinny HIP GEMM
(`dense`): they are launch-latency bound, where it beats the library GEMM by 4-15 us per call on
MI355X; larger ones at <= 64 rows are bandwidth bound and the library GEMM is as fast there."""


def _dense_wide_rows(rows: int, w: torch.Tensor) -> bool:
    """65..256 rows: the skinny GEMM's row groups beat the library GEMM's default solution on
    2048..4096 output rows with K >= 1024 (measured at 192 rows: [4096, 8192] 47 against 61 us,
    [4096, 1024] 10.2 against 11.4 us), where the default tiles leave most of the GPU idle; wider
    N stays on the library GEMM (the 192-row LM head: 881 against 494 us). A K >= 8192 shape
    with a tuned library solution goes back to the library (`blas_tune`: 34.5 us at [4096, 8192])."""
    n, k = w.shape
    if not (64 < rows <= dense.MAX_ROWS and 2048 <= n <= 4096 and k >= 1024):
        return False
    return not (k >= 8192 and blas_tune.prefers_library(rows, n, k))


FUSED_ARGMAX_ROWS = 192
"""Greedy LM-head rows up to which `next_tokens` runs the GEMM with the argmax in its epilogue
(the logits never reach memory). Measured on [M, 4096] x [248320, 4096] bf16 against the
library GEMM + the argmax kernel: 390 against 401 us at 16 rows (skinny tiles), 404 against 423
us at 48 and 427 against 433 us at 64 on the skinny tiles, which the wide form's 512-row tiles
then took to 372-374 us from 17 to 64 rows, and at 192 rows (the wide form's 256-row tiles)
506.5 against 519-520 us (hipBLASLt or rocBLAS, graph replay over two weight copies)."""


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """`F.linear(x, w)`; the shapes the skinny GEMM streams faster run on `dense.linear`."""
    if dense.fits(x, w):
        rows = x.numel() // x.shape[-1]
        if rows <= 64 and w.numel() * w.element_size() <= SMALL_WEIGHT_BYTES:
            return dense.linear(x, w)
        if _dense_wide_rows(rows, w):
            return dense.linear(x, w)
    return F.linear(x, w)


def swiglu(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """`down(silu(gate(x)) * up(x))` with `w_gate_up = cat([gate; up])` (`model.py:638-649`); the
    gate/up GEMM and its SiLU product are one launch when the skinny GEMM takes the shapes."""
    if w_gate_up.numel() * w_gate_up.element_size() <= SMALL_WEIGHT_BYTES and dense.fits(x, w_gate_up):
        act = dense.silu_linear(x, w_gate_up)  # at 192 rows 19 us against 16 us + the SiLU product
    else:
        gate, up = F.linear(x, w_gate_up).chunk(2, dim=-1)
        act = F.silu(gate) * up
    return linear(act, w_down)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3.5 RMSNorm: normalise in fp32, scale by `1 + w` (`model.py:587-604`). Contiguous
    device tensors take the row-norm kernel (`rownorm.rmsnorm`)."""
    if x.device.type == "cuda" and x.is_contiguous():
        return rownorm.rmsnorm(x, w, eps)
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (y * (1.0 + w.float())).to(x.dtype)


def add_rmsnorm(x: torch.Tensor, res: torch.Tensor, w: torch.Tensor,
                eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """`s = x + res`, then `rmsnorm(s, w, eps)`: returns `(s, normed)`; one row-norm launch for
    contiguous device tensors."""
    if x.device.type == "cuda" and x.is_contiguous() and res.is_contiguous():
        return rownorm.add_rmsnorm(x, res, w, eps)
    s = x + res
    return s, rmsnorm(s, w, eps)


def gated_rmsnorm(x: torch.Tensor, gate: torch.Tensor, w: torch.Tensor, eps: float,
                  dtype: torch.dtype) -> torch.Tensor:
    """DeltaNet output norm: RMS-normalise, scale by `w` (no +1), times `silu(gate)`
    (`model.py:613-619`). `x`, `gate` `[..., heads, dim]`; device tensors take the row-norm
    kernel."""
    if x.device.type == "cuda":
        x = x if x.stride(-1) == 1 else x.contiguous()
        gate = gate if gate.stride(-1) == 1 else gate.contiguous()
        return rownorm.gated_rmsnorm(x, gate, w, eps, dtype)
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()
    return (y * F.silu(gate.float())).to(dtype)


def l2norm(x: torch.Tensor, eps: float = 1e-6, scale: float = 1.0) -> torch.Tensor:
    """`x * rsqrt(sum(x^2) + eps) * scale` over the last dim of fp32 `[..., heads, dim]`."""
    if x.device.type == "cuda":
        return rownorm.l2norm(x if x.stride(-1) == 1 else x.contiguous(), eps, scale)
    y = x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)
    return y * scale if scale != 1.0 else y


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE on the first `rot_dim` channels of the last axis (`model.py:631-635`);
    `cos`/`sin` broadcast against `x[..., :rot_dim]`."""
    r = cos.shape[-1]
    rot, rest = x[..., :r].float(), x[..., r:]
    h = r // 2
    turned = torch.cat((-rot[..., h:], rot[..., :h]), dim=-1)
    return torch.cat(((rot * cos + turned * sin).to(x.dtype), rest), dim=-1)


def rope_table(cfg: Cfg, positions: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 `cos`, `sin` `[positions, rot_dim]` (`model.py:2396-2418`)."""
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.rot_dim, 2, device=device).float() / cfg.rot_dim))
    pos = torch.arange(positions, device=device).float()
    ang = pos[:, None] * inv[None, :]
    emb = torch.cat((ang, ang), dim=-1)
    return emb.cos(), emb.sin()


def causal_conv_rows(window: torch.Tensor, weight: torch.Tensor, t: int) -> torch.Tensor:
    """Depthwise causal conv + SiLU over `t` new columns. `window` is `[B, C, conv_k - 1 + t]`
    (the stored window, then the new raw inputs), `weight` `[C, conv_k]`; returns fp32
    `[B, C, t]`. Taps are summed in a fixed order per element, so a row's value does not
    depend on how many rows are computed together (`model.py:2631-2636`)."""
    kk = weight.shape[-1]
    w = weight.float()
    win = window.float()
    acc = win[:, :, 0:t] * w[None, :, 0:1]
    for j in range(1, kk):
        acc = acc + win[:, :, j : j + t] * w[None, :, j : j + 1]
    return F.silu(acc)


def delta_rule_step(state: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    g: torch.Tensor, beta: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """One gated delta-rule step for every (slot, head) (`model.py:651-697`):
    `S <- exp(g) S;  S <- S + k ((v - S^T k) beta)^T;  out = S^T q`. `state` `[B, H, dk, dv]`
    fp32, `q`/`k` `[B, H, dk]` (normalised), `v` `[B, H, dv]`, `g`/`beta` `[B, H]`. Returns the
    new state and `out` `[B, H, dv]`; the input state is not modified."""
    s = state * g.exp()[..., None, None]
    mem = torch.einsum("bhkv,bhk->bhv", s, k)
    delta = (v - mem) * beta[..., None]
    s = s + k[..., :, None] * delta[..., None, :]
    out = torch.einsum("bhkv,bhk->bhv", s, q)
    return s, out


def paged_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                    block_table: torch.Tensor, base_pos: torch.Tensor, ctx_blocks: int,
                    block_size: int, scale: float) -> torch.Tensor:
    """Causal attention of `t` new query rows per lane over the paged cache
    (`verify_attention_paged`, `model.py:1120-1205`). `q` `[B, heads, t, hd]`; the pools (K
    `[rows, kv_heads, hd]`, V `[rows / block, kv_heads, hd, block]`, see `attention.v_blocks`)
    already hold this round's rows; query row `s` of lane `b` sits at
    `base_pos[b] + s` and sees every cached position up to its own. `ctx_blocks` bounds the
    gather (a host value, at least every lane's block count). fp32 math, q's dtype out. bf16
    device tensors with 16-row blocks and head_dim 64/128/256 go to the HIP kernel
    (`attention.paged_attention`: bf16 MFMA, bf16 probabilities, fp32 softmax)."""
    if attention.supported(q, block_size):
        return attention.paged_attention(q, k_pool, v_pool, block_table, base_pos, ctx_blocks * block_size,
                                         scale)
    b, heads, t, hd = q.shape
    kvh = k_pool.shape[1]
    group = heads // kvh
    blocks = block_table[:, :ctx_blocks].long()
    tok = torch.arange(block_size, device=q.device)
    rows = (blocks[:, :, None] * block_size + tok).reshape(b, -1)  # [B, S]
    s_len = rows.shape[1]
    keys = k_pool[rows].float().permute(0, 2, 3, 1).contiguous()  # [B, kvh, hd, S]
    vals = attention.read_v(v_pool, rows).float().permute(0, 2, 1, 3).contiguous()  # [B, kvh, S, hd]
    qg = q.float().reshape(b, kvh, group * t, hd)
    scores = torch.matmul(qg, keys) * scale  # [B, kvh, group*t, S]
    qpos = base_pos.long()[:, None] + torch.arange(t, device=q.device)[None, :]  # [B, t]
    live = torch.arange(s_len, device=q.device)[None, None, :] <= qpos[:, :, None]  # [B, t, S]
    live = live[:, None, None].expand(b, 1, group, t, s_len).reshape(b, 1, group * t, s_len)
    probs = scores.masked_fill(~live, float("-inf")).softmax(-1)
    out = torch.matmul(probs, vals)  # [B, kvh, group*t, hd]
    return out.reshape(b, heads, t, hd).to(q.dtype)


def kv_write_in_kernel(model: "Model") -> bool:
    """Whether this round's K/V rows go to the caches through `attention.kv_write` (a bf16
    model on a device), so that callers need not compute the rows' physical pool rows."""
    return model.device.type == "cuda" and model.dtype == torch.bfloat16


def table_rows(block_table: torch.Tensor, pos: torch.Tensor, block_size: int) -> torch.Tensor:
    """Physical pool rows `block * block_size + pos % block_size` of positions `pos` `[B, t]`
    through per-row block tables `block_table` `[B, blocks]` (`graph_mtp.py:857-860`)."""
    blk = torch.gather(block_table.long(), 1, pos.long() // block_size)
    return blk * block_size + pos.long() % block_size


def fuse_qkv(w: dict) -> dict:
    """Stack an attention layer's q (with its gate rows), k and v projections into one weight
    `qkv_proj` (one GEMM for all three) and re-point `q_proj`, `k_proj`, `v_proj` and `kv_proj`
    at row slices of it; returns `w`."""
    q, k, v = w["q_proj"], w["k_proj"], w["v_proj"]
    qkv = torch.cat([q, k, v])
    a, b = q.shape[0], q.shape[0] + k.shape[0]
    w.update(qkv_proj=qkv, q_proj=qkv[:a], k_proj=qkv[a:b], v_proj=qkv[b:], kv_proj=qkv[a:])
    return w


def split_kv(kv: torch.Tensor, kv_heads: int, head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """k and v `[..., kv_heads, head_dim]` views of a `kv_proj` output `[..., 2 kv_heads hd]`."""
    kd = kv_heads * head_dim
    lead = kv.shape[:-1]
    return kv[..., :kd].view(*lead, kv_heads, head_dim), kv[..., kd:].view(*lead, kv_heads, head_dim)


def gated_attention(model: "Model", w: dict, pool: dict, h: torch.Tensor, base_pos: torch.Tensor,
                    write_rows: torch.Tensor, block_table: torch.Tensor, ctx_blocks: int,
                    keep: torch.Tensor | None = None,
                    positions: torch.Tensor | None = None) -> torch.Tensor:
    """Gated GQA attention of `t` rows per lane (`h` `[B, t, hidden]`, normed): q/gate
    projection, q/k RMSNorm, partial RoPE at `base_pos + s`, this round's K/V written at
    `write_rows` `[B, t]` of `pool`, causal paged attention, `o_proj(out * sigmoid(gate))`
    (`model.py:2158-2290`, `model.py:3519-3577`; the MTP layer's `_attn_rows`, `mtp.py:233-279`,
    is the same call on its own pool). When `kv_write_in_kernel(model)`, `write_rows` may be
    None: the K/V write maps positions to pool rows through `block_table` itself. `keep`
    `[B, t]` bool (optional) masks the K/V writes: rows with False write nothing (on the torch
    path they write into row 0, which lies in the reserved block 0 that no lane owns).
    `positions` `[B, t]` (optional) is `base_pos[:, None] + arange(t)` precomputed. A layer with
    `qkv_proj` (`fuse_qkv`) projects q, gate, k and v with one GEMM."""
    c = model.cfg
    b, t, _ = h.shape
    if "qkv_proj" in w:
        qd = 2 * c.heads * c.head_dim
        qkv = linear(h, w["qkv_proj"])
        qg = qkv[..., :qd].view(b, t, c.heads, 2 * c.head_dim)
        kp, v = split_kv(qkv[..., qd:], c.kv_heads, c.head_dim)
    else:
        qg = F.linear(h, w["q_proj"]).view(b, t, c.heads, 2 * c.head_dim)
        kp = linear(h, w["k_proj"]).view(b, t, c.kv_heads, c.head_dim)
        v = linear(h, w["v_proj"]).view(b, t, c.kv_heads, c.head_dim)
    q, gate = qg[..., : c.head_dim], qg[..., c.head_dim :]
    if positions is not None:
        pos = positions
    elif t == 1:
        pos = base_pos.long()[:, None]
    else:
        pos = base_pos.long()[:, None] + torch.arange(t, device=h.device)[None, :]
    if h.device.type == "cuda":  # q/k norm and RoPE in one row-norm launch each
        rope = (model.cos, model.sin, pos.reshape(-1))
        q = rownorm.rmsnorm(q, w["q_norm"], c.eps, heads=True, rope=rope)
        k = rownorm.rmsnorm(kp, w["k_norm"], c.eps, heads=True, rope=rope)
    else:
        q, k = rmsnorm(q, w["q_norm"], c.eps), rmsnorm(kp, w["k_norm"], c.eps)
        cos, sin = model.cos[pos][:, :, None], model.sin[pos][:, :, None]  # [B, t, 1, rot]
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    if kv_write_in_kernel(model):  # positions -> pool rows through the table, inside the kernel
        attention.kv_write(pool["k"], pool["v"], k, v, block_table, base_pos, keep)
    else:
        rows = write_rows.reshape(-1).long()
        if keep is not None:
            rows = torch.where(keep.reshape(-1), rows, torch.zeros_like(rows))
        pool["k"][rows] = k.reshape(-1, c.kv_heads, c.head_dim)
        attention.write_v(pool["v"], rows, v.reshape(-1, c.kv_heads, c.head_dim))
    if attention.supported(q, c.block_size):
        # q read in its [B, t, heads, hd] layout, the sigmoid gate applied in the epilogue
        out = attention.paged_attention_gated(q, pool["k"], pool["v"], block_table, base_pos,
                                              ctx_blocks * c.block_size, c.head_dim ** -0.5, gate)
        return linear(out.reshape(b, t, -1), w["o_proj"])
    out = paged_attention(q.transpose(1, 2), pool["k"], pool["v"], block_table, base_pos, ctx_blocks,
                          c.block_size, c.head_dim ** -0.5)
    out = out.transpose(1, 2).reshape(b, t, -1)
    return F.linear(out * torch.sigmoid(gate.reshape(b, t, -1)), w["o_proj"])


# ---------------------------------------------------------------- paged KV block tables


class BlockTables:
    """Per-lane block tables over one pool of `block_size`-row blocks (`block_pool.py`'s role).

    Block 0 is never handed out: unused table entries point at it, so a padded read stays in
    bounds and reads rows no lane owns (`block_pool.py:38`). Blocks are handed out in a seeded
    shuffled order so that a lane's physical rows are not contiguous.
    """

    def __init__(self, lanes: int, max_seq: int, block_size: int, device: torch.device,
                 seed: int = 0) -> None:
        self.lanes, self.block_size = lanes, block_size
        self.max_blocks = (max_seq + block_size - 1) // block_size
        self.n_blocks = lanes * self.max_blocks + 1
        gen = torch.Generator().manual_seed(seed)
        self._free = (torch.randperm(self.n_blocks - 1, generator=gen) + 1).tolist()
        self.host = [[] for _ in range(lanes)]
        self.held_positions = [0] * lanes  # len(host[lane]) * block_size
        self.table = torch.zeros(lanes, self.max_blocks, dtype=torch.int32, device=device)
        self.device = device

    @property
    def rows(self) -> int:
        return self.n_blocks * self.block_size

    def grow(self, lane: int, length: int) -> None:
        """Make lane `lane` hold at least `length` positions (idempotent below that)."""
        need = (length + self.block_size - 1) // self.block_size
        if need > self.max_blocks:
            raise ValueError(f"lane {lane}: {length} positions exceed the table's {self.max_blocks} blocks")
        have = self.host[lane]
        if need <= len(have):
            return
        new = [self._free.pop() for _ in range(need - len(have))]
        self.table[lane, len(have) : need] = torch.tensor(new, dtype=torch.int32).to(self.device)
        have.extend(new)
        self.held_positions[lane] = len(have) * self.block_size

    def grow_many(self, lanes, lengths) -> None:
        """`grow` for several lanes with one host-to-device copy and one scatter for every new
        table entry (per-lane copies from pageable memory each wait for the stream). A call in
        which every lane already holds its blocks is one pass of builtin comparisons."""
        cap = self.held_positions
        pairs = list(zip(lanes, lengths, strict=True))
        if all(int(n) <= cap[int(lane)] for lane, n in pairs):
            return
        needs = []
        for lane, length in pairs:
            need = (int(length) + self.block_size - 1) // self.block_size
            if need > self.max_blocks:
                raise ValueError(f"lane {lane}: {length} positions exceed the table's {self.max_blocks} blocks")
            needs.append((int(lane), need))
        upd = []
        for lane, need in needs:
            have = self.host[lane]
            for col in range(len(have), need):
                blk = self._free.pop()
                have.append(blk)
                upd.append((lane, col, blk))
            cap[lane] = len(have) * self.block_size
        if not upd:
            return
        pin = self.table.is_cuda
        u = torch.tensor(upd, dtype=torch.long, pin_memory=pin).to(self.device, non_blocking=pin)
        self.table[u[:, 0], u[:, 1]] = u[:, 2].to(torch.int32)

    def release(self, lane: int) -> None:
        self._free.extend(reversed(self.host[lane]))
        self.host[lane] = []
        self.held_positions[lane] = 0
        self.table[lane].zero_()

    def physical_rows(self, lanes: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """Physical pool rows of positions `pos` `[B, t]` of lanes `lanes` `[B]` (device)."""
        return table_rows(self.table[lanes.long()], pos, self.block_size)


# ---------------------------------------------------------------- weights


def _normal(shape, std, dtype, device, gen) -> torch.Tensor:
    """N(0, std) drawn on the generator's device, stored as `dtype` on `device`."""
    return (torch.randn(*shape, generator=gen, device=gen.device, dtype=torch.float32) * std).to(device, dtype)


def random_experts(cfg: Cfg, device: torch.device, gen: torch.Generator, mode: str) -> dict:
    """MXFP4 expert payloads in the `load_experts` layout (`model.py:758-804`): `gate_up`
    `[E, 2I, H/2]` (gate rows then up rows), `down` `[E, H, I/2]`, e8m0 scales per 32.

    `mode="quantized"`: fp32 N(0, 0.02) weights quantised with `mxfp4.quantize_mxfp4`.
    `mode="bytes"`: packed bytes uniform over 0..255 and scale bytes uniform over 118..130.
    `mode="dense"`: bf16 N(0, 0.02) `gate_up` `[E, 2I, H]` and `down` `[E, H, I]`, the layout of
    the real checkpoint's MTP layer (its experts are not quantised).
    """
    e, i, h = cfg.experts, cfg.inter, cfg.hidden
    if mode == "dense":
        return {"gate_up": _normal((e, 2 * i, h), 0.02, torch.bfloat16, device, gen),
                "down": _normal((e, h, i), 0.02, torch.bfloat16, device, gen)}
    if mode == "quantized":
        gu = _normal((e * 2 * i, h), 0.02, torch.float32, gen.device, gen)
        dn = _normal((e * h, i), 0.02, torch.float32, gen.device, gen)
        gq, gs = mxfp4.quantize_mxfp4(gu)
        dq, ds = mxfp4.quantize_mxfp4(dn)
        parts = {"gate_up": gq.view(e, 2 * i, h // 2), "gate_up_scale": gs.view(e, 2 * i, h // 32),
                 "down": dq.view(e, h, i // 2), "down_scale": ds.view(e, h, i // 32)}
        return {name: ten.to(device) for name, ten in parts.items()}
    if mode != "bytes":
        raise ValueError(f"unknown expert init {mode!r}")

    def u8(shape, lo, hi):
        return torch.randint(lo, hi + 1, shape, generator=gen, device=gen.device,
                             dtype=torch.int32).to(device, torch.uint8)

    return {"gate_up": u8((e, 2 * i, h // 2), 0, 255), "gate_up_scale": u8((e, 2 * i, h // 32), 118, 130),
            "down": u8((e, h, i // 2), 0, 255), "down_scale": u8((e, h, i // 32), 118, 130)}


def attention_weights(cfg: Cfg, dtype, device, gen) -> dict:
    qd, kd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    return fuse_qkv({
        "q_proj": _normal((2 * qd, cfg.hidden), 0.02, dtype, device, gen),  # per head: q then gate
        "k_proj": _normal((kd, cfg.hidden), 0.02, dtype, device, gen),
        "v_proj": _normal((kd, cfg.hidden), 0.02, dtype, device, gen),
        "o_proj": _normal((cfg.hidden, qd), 0.02, dtype, device, gen),
        "q_norm": _normal((cfg.head_dim,), 0.02, dtype, device, gen),
        "k_norm": _normal((cfg.head_dim,), 0.02, dtype, device, gen),
    })


def deltanet_weights(cfg: Cfg, dtype, device, gen) -> dict:
    vh = cfg.v_heads
    a_log = torch.log(torch.rand(vh, generator=gen, device=gen.device) * 15.0 + 1.0).to(device)
    return {
        "in_proj_all": _normal((sum(cfg.in_proj_sizes), cfg.hidden), 0.02, dtype, device, gen),
        "conv": _normal((cfg.conv_dim, cfg.conv_k), 0.2, dtype, device, gen),
        "A_log": a_log.float(),
        "dt_bias": torch.rand(vh, generator=gen, device=gen.device).to(device),
        "dn_norm": (1.0 + _normal((cfg.v_dim,), 0.02, torch.float32, device, gen)).to(dtype),
        "out_proj": _normal((cfg.hidden, vh * cfg.v_dim), 0.02, dtype, device, gen),
    }


def moe_weights(cfg: Cfg, dtype, device, gen, expert_mode: str) -> dict:
    return {
        # router rows, then the shared expert's gate row (`model.py:2811-2843`)
        "router_gate": _normal((cfg.experts + 1, cfg.hidden), 0.02, dtype, device, gen),
        "shared_gate_up": _normal((2 * cfg.shared_inter, cfg.hidden), 0.02, dtype, device, gen),
        "shared_down": _normal((cfg.hidden, cfg.shared_inter), 0.02, dtype, device, gen),
        "experts": random_experts(cfg, device, gen, expert_mode),
    }


# ---------------------------------------------------------------- the model


@dataclass
class DeltaNetRows:
    """What `deltanet_commit` needs from a verify forward of one DeltaNet layer: the raw
    conv inputs and the per-row recurrence inputs, `[B, t, ...]`."""

    raw_qkv: torch.Tensor  # [B, conv_dim, t], model dtype (a view of `proj` on a device)
    q: torch.Tensor  # [B, t, k_heads, k_dim] fp32, normalised and scaled
    k: torch.Tensor  # [B, t, k_heads, k_dim] fp32, normalised
    v: torch.Tensor  # [B, t, v_heads, v_dim] fp32
    g: torch.Tensor  # [B, t, v_heads] fp32
    beta: torch.Tensor  # [B, t, v_heads] fp32
    proj: torch.Tensor | None = None  # [B, t, P] in-projection output (device path)


@dataclass
class VerifyOut:
    """A forward over `[B, t]` fed tokens: the raw (pre-final-norm) hidden states and, per
    DeltaNet layer, the rows its commit replays."""

    hidden: torch.Tensor
    dn_rows: dict[int, DeltaNetRows] = field(default_factory=dict)
    normed: torch.Tensor | None = None  # the final-normed rows, when asked for


class Model:
    """The target stack with its per-slot state. `lanes` is the slot-pool size; every call
    takes the slots it works on as a `[B]` list or tensor."""

    def __init__(self, cfg: Cfg, device: torch.device | str = "cpu", dtype: torch.dtype = torch.float32,
                 lanes: int = 2, max_seq: int = 256, seed: int = 0, expert_mode: str = "quantized",
                 moe_rows: int | None = None, init_device: str | None = None) -> None:
        """Random-init weights from `seed`. They are drawn on `init_device` (default: the CPU
        for models below hidden 1024, so a small model has the same weights on every device;
        the model's device otherwise) and stored on `device`. `moe_rows` sizes the routed-MoE
        workspace (rows per call; default `4 * lanes`)."""
        self.cfg, self.dtype = cfg, dtype
        self.device = torch.device(device)
        self.lanes, self.max_seq = lanes, max_seq
        dev = self.device
        gdev = init_device or ("cpu" if cfg.hidden < 1024 else dev)
        gen = torch.Generator(device=gdev).manual_seed(seed)
        self.gen = gen
        self.embed = _normal((cfg.vocab, cfg.hidden), 0.02, dtype, dev, gen)
        self.lm_head = _normal((cfg.vocab, cfg.hidden), 0.02, dtype, dev, gen)
        self.final_norm = _normal((cfg.hidden,), 0.02, dtype, dev, gen)
        self.layers: list[dict] = []
        for ty in cfg.layer_types:
            w = {"in_norm": _normal((cfg.hidden,), 0.02, dtype, dev, gen),
                 "post_norm": _normal((cfg.hidden,), 0.02, dtype, dev, gen)}
            w.update(attention_weights(cfg, dtype, dev, gen) if ty == ATTN else deltanet_weights(cfg, dtype, dev, gen))
            w.update(moe_weights(cfg, dtype, dev, gen, expert_mode))
            self.layers.append(w)
        self.blocks = BlockTables(lanes, max_seq, cfg.block_size, dev, seed)
        self.pool: list[dict] = []
        for ty in cfg.layer_types:
            if ty == ATTN:  # V transposed inside each block (attention.v_blocks)
                shape = (self.blocks.rows, cfg.kv_heads, cfg.head_dim)
                vshape = (self.blocks.rows // cfg.block_size, cfg.kv_heads, cfg.head_dim, cfg.block_size)
                self.pool.append({"k": torch.zeros(shape, dtype=dtype, device=dev),
                                  "v": torch.zeros(vshape, dtype=dtype, device=dev)})
            else:
                self.pool.append({
                    "conv": torch.zeros(lanes, cfg.conv_dim, cfg.conv_k - 1, dtype=dtype, device=dev),
                    "rec": torch.zeros(lanes, cfg.v_heads, cfg.k_dim, cfg.v_dim, dtype=torch.float32, device=dev),
                })
        self.hidden_cache = torch.zeros(lanes, cfg.hidden, dtype=dtype, device=dev)
        self.cos, self.sin = rope_table(cfg, max_seq, dev)
        self.mtp = None
        self.route_log: list | None = None
        """When a list, every MoE call appends `(layer, h, top_i)`: the layer index (or "mtp"), a
        copy of its input rows and its selected experts. A test hook; None in serving."""
        self.moe_ws = None
        if dev.type == "cuda":
            rows = moe_rows or lanes * 4
            self.moe_ws = mxfp4_gemv.moe_scratch(max(rows, 16), cfg.top_k, cfg.experts, cfg.inter,
                                                 cfg.hidden, dev, dtype)

    # ------------------------------------------------------------ blocks

    def lane_index(self, lanes) -> torch.Tensor:
        if torch.is_tensor(lanes):
            return lanes.to(self.device, torch.long)
        return torch.tensor(list(lanes), dtype=torch.long, device=self.device)

    def reset(self, lane: int) -> None:
        """Forget slot `lane`'s sequence: blocks, DeltaNet state and cached hidden."""
        self.blocks.release(lane)
        for ty, p in zip(self.cfg.layer_types, self.pool):
            if ty != ATTN:
                p["conv"][lane].zero_()
                p["rec"][lane].zero_()
        self.hidden_cache[lane].zero_()

    # ------------------------------------------------------------ sublayers

    def moe(self, w: dict, h: torch.Tensor) -> torch.Tensor:
        """Routed MXFP4 experts + gated shared expert over rows `h` `[N, hidden]`
        (`model.py:2811-2873`)."""
        c = self.cfg
        log = self.route_log
        if h.device.type == "cuda" and mxfp4_gemv.available(h.device):
            hc = h.contiguous()
            if mxfp4_gemv.layer_fits(hc, w["router_gate"], w["shared_gate_up"], w["shared_down"],
                                     w["experts"], c.top_k, (0, c.experts)):
                # router, shared expert and routed experts in the routed layer's launches
                routing_out = None
                if log is not None:
                    routing_out = (torch.empty(hc.shape[0], c.top_k, dtype=torch.float32, device=h.device),
                                   torch.empty(hc.shape[0], c.top_k, dtype=torch.int32, device=h.device))
                    log.append((self._layer_of(w), hc.clone(), routing_out[1]))
                return mxfp4_gemv.fused_moe_layer(hc, w["router_gate"], w["shared_gate_up"],
                                                  w["shared_down"], w["experts"], c.top_k, (0, c.experts),
                                                  routing_out=routing_out)
        routing = linear(h, w["router_gate"])
        if h.device.type == "cuda":
            top_w, top_i = router_fused.route(routing, c.experts, c.top_k, index_dtype=torch.int32)
        else:
            probs = routing[:, : c.experts].float().softmax(-1)
            top_w, top_i = probs.topk(c.top_k, dim=-1)
            top_w = top_w / top_w.sum(-1, keepdim=True)
        if log is not None:
            log.append((self._layer_of(w), h.clone(), top_i.clone()))
        assign = (top_i.reshape(-1), top_w.reshape(-1))
        shared = swiglu(h, w["shared_gate_up"], w["shared_down"])
        if "gate_up_scale" not in w["experts"]:
            routed = self._dense_moe(w["experts"], h, top_i, top_w)
        elif mxfp4_gemv.available(h.device):
            # the shared expert's gated term is added inside the routed layer's combine
            return mxfp4_gemv.fused_moe(h.contiguous(), w["experts"], assign, c.top_k, (0, c.experts),
                                        inter=self.moe_ws, shared=shared.contiguous(),
                                        shared_gate=routing[:, c.experts :])
        else:
            # SEED_FUSED_MOE=0 (or the CPU): the torch dequant-then-multiply path of
            # `_routed_grouped` (`model.py:3170-3236`), dequantised by the torch table lookup
            routed = mxfp4_gemv.reference_moe(h, w["experts"], assign, c.top_k, (0, c.experts),
                                              mxfp4.dequant_torch)
        return routed + torch.sigmoid(routing[:, c.experts :]) * shared

    def moe_add_norm(self, w: dict, h: torch.Tensor, x: torch.Tensor,
                     norm_w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """`add_rmsnorm(x, moe(w, h), norm_w)` with `x` of `h`'s rows: `(x + moe, normed)`. On
        a device, where the whole-layer launches take `h`, the residual add and the norm ride in
        the layer's last launch (`mxfp4_gemv.fused_moe_layer(add_norm=)`, the same bits)."""
        c = self.cfg
        rows = h.numel() // h.shape[-1]
        if (h.device.type == "cuda" and self.route_log is None and mxfp4_gemv.available(h.device)
                and x.dtype == torch.bfloat16 and norm_w.dtype == torch.bfloat16
                and mxfp4_gemv.add_norm_supported(rows, c.hidden)):
            hc = h.reshape(rows, -1).contiguous()
            if mxfp4_gemv.layer_fits(hc, w["router_gate"], w["shared_gate_up"], w["shared_down"],
                                     w["experts"], c.top_k, (0, c.experts)):
                s, n = mxfp4_gemv.fused_moe_layer(
                    hc, w["router_gate"], w["shared_gate_up"], w["shared_down"], w["experts"],
                    c.top_k, (0, c.experts),
                    add_norm=(x.reshape(rows, -1).contiguous(), norm_w.contiguous(), c.eps))
                return s.view(x.shape), n.view(x.shape)
        return add_rmsnorm(x, self.moe(w, h.reshape(rows, -1)).view(x.shape), norm_w, c.eps)

    def _layer_of(self, w: dict):
        for i, lw in enumerate(self.layers):
            if lw is w:
                return i
        return "mtp"

    def _dense_moe(self, ex: dict, h: torch.Tensor, top_i: torch.Tensor,
                   top_w: torch.Tensor) -> torch.Tensor:
        """Routed dense (bf16) experts: `mtp_dense_moe.fused_moe` on a device, the per-expert
        torch form of `mtp._routed_grouped` (`mtp.py:347-388`) on the CPU."""
        c = self.cfg
        if h.device.type == "cuda":
            return mtp_dense_moe.fused_moe(h.to(torch.bfloat16).contiguous(), ex, (top_i, top_w),
                                           c.top_k, (0, c.experts)).to(h.dtype)
        out = torch.zeros(h.shape[0], ex["down"].shape[1], dtype=torch.float32)
        flat_i, flat_w = top_i.reshape(-1), top_w.reshape(-1).float()
        tok = torch.arange(flat_i.numel()) // c.top_k
        for e in flat_i.unique().tolist():
            sel = (flat_i == e).nonzero()[:, 0]
            gate, up = (h[tok[sel]].float() @ ex["gate_up"][e].float().T).chunk(2, dim=-1)
            y = (F.silu(gate) * up) @ ex["down"][e].float().T
            out.index_add_(0, tok[sel], y * flat_w[sel, None])
        return out.to(h.dtype)

    def attention_rows(self, w: dict, pool: dict, h: torch.Tensor, lanes: torch.Tensor,
                       base_pos: torch.Tensor, ctx_len: int, block_table: torch.Tensor | None = None,
                       keep: torch.Tensor | None = None,
                       positions: torch.Tensor | None = None) -> torch.Tensor:
        """Gated GQA attention for `t` rows per lane at positions `base_pos + s` (`attn_verify`,
        `model.py:3519-3577`) over `block_table` `[B, blocks]` (default: the lanes' own tables),
        K/V writes masked by `keep` `[B, t]`. `ctx_len` is a host bound on `base_pos + t`;
        `positions` (optional) the `[B, t]` positions precomputed."""
        c = self.cfg
        t = h.shape[1]
        table = self.blocks.table[lanes] if block_table is None else block_table
        rows = None
        if not kv_write_in_kernel(self):
            pos = base_pos.long()[:, None] + torch.arange(t, device=h.device)[None, :]
            rows = table_rows(table, pos, c.block_size)
        ctx_blocks = (ctx_len + c.block_size - 1) // c.block_size
        return gated_attention(self, w, pool, h, base_pos, rows, table, ctx_blocks, keep, positions)

    def deltanet_verify(self, w: dict, pool: dict, h: torch.Tensor,
                        lanes: torch.Tensor) -> tuple[torch.Tensor, DeltaNetRows]:
        """Gated DeltaNet over `t` rows per lane from the committed state, which is read and
        not written (`deltanet_verify`, `model.py:3738-3905`)."""
        c = self.cfg
        b, t, _ = h.shape
        proj = F.linear(h, w["in_proj_all"])
        qkv, z, b_raw, a_raw = proj.split(c.in_proj_sizes, dim=-1)
        raw = qkv.transpose(1, 2)  # [B, C, t]
        if h.device.type == "cuda":
            # conv, SiLU, split, q/k norms, g and beta in one launch; then the recurrence
            q, k, v, g, beta = deltanet.prep(proj, pool["conv"], lanes, w["conv"], w["A_log"],
                                             w["dt_bias"], c.k_heads, c.k_dim, c.v_heads, c.v_dim)
            out = deltanet.delta_rule(pool["rec"], lanes, q, k, v, g, beta)  # [B, t, vh, vd] fp32
            normed = gated_rmsnorm(out, z.reshape(b, t, c.v_heads, c.v_dim), w["dn_norm"], c.eps, h.dtype)
            mixer = linear(normed.reshape(b, t, -1), w["out_proj"])
            return mixer, DeltaNetRows(raw, q, k, v, g, beta, proj)
        window = torch.cat([pool["conv"][lanes], raw], dim=-1)
        mixed = causal_conv_rows(window, w["conv"], t).to(h.dtype).transpose(1, 2)  # [B, t, C]
        kd = c.k_heads * c.k_dim
        q = mixed[..., :kd].reshape(b, t, c.k_heads, c.k_dim).float()
        k = mixed[..., kd : 2 * kd].reshape(b, t, c.k_heads, c.k_dim).float()
        v = mixed[..., 2 * kd :].reshape(b, t, c.v_heads, c.v_dim).float()
        q = l2norm(q, scale=c.k_dim ** -0.5)  # [B, t, k_heads, k_dim]; v head h reads k head h // rep
        k = l2norm(k)
        beta = torch.sigmoid(b_raw.float())
        g = -w["A_log"].float().exp() * F.softplus(a_raw.float() + w["dt_bias"].float())
        rep = c.v_heads // c.k_heads
        qe, ke = q.repeat_interleave(rep, dim=2), k.repeat_interleave(rep, dim=2)
        state = pool["rec"][lanes]
        outs = []
        for s in range(t):
            state, o = delta_rule_step(state, qe[:, s], ke[:, s], v[:, s], g[:, s], beta[:, s])
            outs.append(o)
        out = torch.stack(outs, dim=1)  # [B, t, vh, vd] fp32
        normed = gated_rmsnorm(out, z.reshape(b, t, c.v_heads, c.v_dim), w["dn_norm"], c.eps, h.dtype)
        mixer = F.linear(normed.reshape(b, t, -1), w["out_proj"])
        return mixer, DeltaNetRows(raw.contiguous(), q, k, v, g, beta)

    def deltanet_commit(self, pool: dict, rows: DeltaNetRows, lanes: torch.Tensor,
                        lengths: torch.Tensor, conv_idx: torch.Tensor | None = None,
                        active: torch.Tensor | None = None) -> None:
        """Advance slot `lanes[j]`'s conv window and recurrent state by `lengths[j]` of the
        verified rows (1..t) (`deltanet_verify_rollback`, `model.py:3907-3972`). `conv_idx`
        `[B, conv_k - 1]`, when given, is the acceptance kernel's window index
        `min(lengths + w, conv_k - 2 + t)`; it is computed here otherwise. Rows with `active`
        False (padding) leave every slot as it is."""
        c = self.cfg
        k1 = c.conv_k - 1
        t = rows.q.shape[1]
        n = lengths.to(self.device, torch.long)
        if conv_idx is not None:
            idx = conv_idx.long()
        else:
            idx = (n[:, None] + torch.arange(k1, device=self.device)[None, :]).clamp(max=k1 + t - 1)
        if self.device.type == "cuda":
            # the kernels skip a row whose slot lies outside the pool: padding commits nothing
            slots = lanes if active is None else torch.where(active, lanes, torch.full_like(lanes, -1))
            if rows.proj is not None:  # the state and the conv window in one launch
                deltanet.commit(pool["rec"], pool["conv"], slots, rows.q, rows.k, rows.v, rows.g,
                                rows.beta, n, rows.proj, idx, c.conv_dim)
                return
            window = torch.cat([pool["conv"][lanes], rows.raw_qkv], dim=-1)  # [B, C, k1 + t]
            new = torch.gather(window, 2, idx[:, None, :].expand(-1, window.shape[1], -1))
            if active is not None:
                new = torch.where(active[:, None, None], new, pool["conv"][lanes])
            pool["conv"][lanes] = new
            deltanet.delta_rule(pool["rec"], slots, rows.q, rows.k, rows.v, rows.g, rows.beta, n,
                                want_out=False)
            return
        window = torch.cat([pool["conv"][lanes], rows.raw_qkv], dim=-1)  # [B, C, k1 + t]
        conv = torch.gather(window, 2, idx[:, None, :].expand(-1, window.shape[1], -1))
        rep = c.v_heads // c.k_heads
        qe, ke = rows.q.repeat_interleave(rep, dim=2), rows.k.repeat_interleave(rep, dim=2)
        state = pool["rec"][lanes]
        for s in range(t):
            nxt, _ = delta_rule_step(state, qe[:, s], ke[:, s], rows.v[:, s], rows.g[:, s], rows.beta[:, s])
            state = torch.where((s < n)[:, None, None, None], nxt, state)
        sel = torch.arange(lanes.shape[0]) if active is None else active.nonzero()[:, 0]
        pool["conv"][lanes[sel]] = conv[sel]
        pool["rec"][lanes[sel]] = state[sel]

    # ------------------------------------------------------------ forward

    def forward_rows(self, ids: torch.Tensor, lanes, base_pos: torch.Tensor, ctx_len: int, *,
                     block_table: torch.Tensor | None = None,
                     active: torch.Tensor | None = None,
                     positions: torch.Tensor | None = None,
                     final_norm: bool = False) -> VerifyOut:
        """The wide forward over fed tokens `ids` `[B, t]` at positions `base_pos[b] + s`
        (`verify_and_commit`'s layer loop, `mtp.py:767-772`). Writes the rows' K/V; DeltaNet
        state is left for `commit`. `ctx_len` is a host bound on `max(base_pos) + t`.

        `block_table` `[B, blocks]` (a round buffer's, `graph_mtp.py:141-178`) replaces the
        lanes' own tables for the attention reads and the K/V writes; rows with `active` False
        (padding) read their slot's state but write no K/V. `positions` (optional) is
        `base_pos[:, None] + arange(t)` precomputed (a round buffer's `pos_grid`). With
        `final_norm`, `res.normed` also holds the final-normed rows (the last residual add and
        the norm in one launch)."""
        c = self.cfg
        lanes = self.lane_index(lanes)
        base_pos = base_pos.to(self.device, torch.long)
        keep = None if active is None else active[:, None].expand(ids.shape[0], ids.shape[1])
        x = self.embed[ids.to(self.device)]
        res = VerifyOut(x)
        n_layers = len(c.layer_types)
        h = rmsnorm(x, self.layers[0]["in_norm"], c.eps)
        for i, ty in enumerate(c.layer_types):
            w, pool = self.layers[i], self.pool[i]
            if ty == ATTN:
                mixer = self.attention_rows(w, pool, h, lanes, base_pos, ctx_len, block_table, keep,
                                            positions)
            else:
                mixer, rows = self.deltanet_verify(w, pool, h, lanes)
                res.dn_rows[i] = rows
            x, hm = add_rmsnorm(x, mixer, w["post_norm"], c.eps)
            # the MoE output joins the residual stream in front of the next norm (the next
            # layer's input norm, or the final norm): one fused launch where the layer allows
            nxt = self.layers[i + 1]["in_norm"] if i + 1 < n_layers else (self.final_norm if final_norm else None)
            if nxt is None:
                b, t, _ = hm.shape
                x = x + self.moe(w, hm.reshape(b * t, -1)).view(x.shape)
            else:
                x, h = self.moe_add_norm(w, hm, x, nxt)
        res.hidden = x
        if final_norm:
            res.normed = h
        return res

    def commit(self, res: VerifyOut, lanes, lengths: torch.Tensor,
               conv_idx: torch.Tensor | None = None, active: torch.Tensor | None = None) -> None:
        """Advance every DeltaNet layer's state of `lanes` by `lengths` verified rows; rows with
        `active` False (padding) leave their slots untouched."""
        lanes = self.lane_index(lanes)
        if active is not None and self.device.type == "cuda":
            # the kernels skip a row whose slot lies outside the pool: padding commits nothing
            lanes, active = torch.where(active, lanes, torch.full_like(lanes, -1)), None
        for i, rows in res.dn_rows.items():
            self.deltanet_commit(self.pool[i], rows, lanes, lengths, conv_idx, active)

    def unembed(self, normed: torch.Tensor) -> torch.Tensor:
        return F.linear(normed, self.lm_head)

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.unembed(rmsnorm(hidden, self.final_norm, self.cfg.eps))

    def fused_argmax(self, rows: int, normed: torch.Tensor) -> bool:
        """Whether `next_tokens` takes the GEMM with the argmax epilogue for these rows."""
        return rows <= FUSED_ARGMAX_ROWS and dense.fits(normed, self.lm_head)

    def next_tokens(self, normed: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """Greedy next token of final-normed rows `[..., hidden]`: `argmax(unembed(normed))`.
        Up to FUSED_ARGMAX_ROWS bf16 device rows take the GEMM with its argmax epilogue (the
        logits never reach memory; same first-occurrence rule over the bf16 logits,
        `mtp.py:640-658`). `out` (optional, int64 of the leading shape) receives the ids."""
        rows = normed.numel() // normed.shape[-1]
        if self.fused_argmax(rows, normed):
            return dense.argmax_linear(normed, self.lm_head, out)
        ids = self.argmax(self.unembed(normed))
        return ids if out is None else out.copy_(ids.view(out.shape))

    def argmax(self, logits: torch.Tensor) -> torch.Tensor:
        """First-occurrence argmax over the vocab (the HIP kernel on a device)."""
        if logits.device.type == "cuda":
            import mtp as mtp_mod

            return mtp_mod.argmax_rows(logits)
        return logits.float().argmax(-1)

    def cached_hidden(self, lane: int) -> torch.Tensor:
        return self.hidden_cache[lane : lane + 1]

    def cache_hidden(self, lane: int, h: torch.Tensor) -> None:
        self.hidden_cache[lane].copy_(h.reshape(-1))

    # ------------------------------------------------------------ sequence entry points

    def prefill(self, lane: int, tokens: list[int]) -> torch.Tensor:
        """Run a prompt into slot `lane` from position 0; returns the last row's logits
        `[vocab]` and leaves the slot's state, the MTP cache and the cached hidden after the
        whole prompt."""
        t = len(tokens)
        self.reset(lane)
        self.blocks.grow(lane, t)
        ids = torch.tensor([tokens], dtype=torch.long, device=self.device)
        base = torch.zeros(1, dtype=torch.long, device=self.device)
        res = self.forward_rows(ids, [lane], base, t)
        self.commit(res, [lane], torch.tensor([t], device=self.device))
        if self.mtp is not None:
            import mtp as mtp_mod

            previous = torch.cat([torch.zeros_like(res.hidden[:, :1]), res.hidden[:, :-1]], dim=1)
            pos = torch.arange(t, device=self.device)[None, :]
            rows = self.blocks.physical_rows(self.lane_index([lane]), pos)
            mtp_mod.cache_target_rows(self, self.mtp, ids, previous, pos, rows)
        self.cache_hidden(lane, res.hidden[0, -1])
        return self.logits(res.hidden[0, -1:])[0]

    def decode(self, lanes: list[int], tokens: list[int], positions: list[int]) -> torch.Tensor:
        """One ordinary decode step: token `tokens[j]` at `positions[j]` of slot `lanes[j]`.
        Returns logits `[B, vocab]`; commits the state and extends the MTP cache."""
        for lane, p in zip(lanes, positions, strict=True):
            self.blocks.grow(lane, p + 1)
        ids = torch.tensor([[tk] for tk in tokens], dtype=torch.long, device=self.device)
        base = torch.tensor(positions, dtype=torch.long, device=self.device)
        res = self.forward_rows(ids, lanes, base, max(positions) + 1)
        lane_t = self.lane_index(lanes)
        self.commit(res, lane_t, torch.ones(len(lanes), dtype=torch.long, device=self.device))
        if self.mtp is not None:
            import mtp as mtp_mod

            previous = self.hidden_cache[lane_t][:, None]
            pos = base[:, None]
            mtp_mod.cache_target_rows(self, self.mtp, ids, previous, pos,
                                      self.blocks.physical_rows(lane_t, pos))
        self.hidden_cache[lane_t] = res.hidden[:, 0]
        return self.logits(res.hidden[:, 0])


def greedy_reference(model: Model, lane: int, token: int, pos: int, n: int) -> list[int]:
    """`n` tokens of plain greedy decode from `token` at `pos` in slot `lane` (the sequential
    baseline a speculative round must reproduce, `test_mtp.py:488-513`)."""
    out = []
    for _ in range(n):
        logits = model.decode([lane], [token], [pos])
        token = int(model.argmax(logits)[0])
        out.append(token)
        pos += 1
    return out

