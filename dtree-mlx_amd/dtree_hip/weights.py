"""Qwen3 target weights in the device layout the verify kernels stream.

Per layer (all bf16, nn.Linear [out, in] layout):
  wqkv [q_dim + 2*kv_dim, H]   rows = q heads | k heads | v heads
  wo   [H, q_dim]
  wgu  [2F, H]                 gate / up interleaved in 16-row groups, so one
                               32-row GEMM tile holds gate and up of the same
                               16 FFN features (fused SwiGLU epilogue)
  wd   [H, F]
  input_norm, post_norm [H], q_norm, k_norm [head_dim]
Global: embed [V, H] (tied LM head), final_norm [H].

Linear weights and the embedding are stored in the GEMM's tiled layout
(DTREE_W_TILED: [N/32][K/64][4][64][8], the order the kernel lanes consume, so
every weight load instruction of a wavefront reads one contiguous kilobyte);
``untile_weight`` restores nn.Linear order for host-side checks.

Random init follows the synthetic workload: linear and embedding weights
N(0, 0.02) in bf16, norm weights 1.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .config import Qwen3Config


W_ROWMAJOR, W_TILED, W_Q4G64, W_TILED_F16 = 0, 1, 2, 3


def tile_weight(w: torch.Tensor) -> torch.Tensor:
    """[n, k] row-major -> DTREE_W_TILED (same shape, permuted storage)."""
    n, k = w.shape
    if n % 32 or k % 64:
        raise ValueError("tiled weights need n % 32 == 0 and k % 64 == 0")
    t = w.reshape(n // 32, 32, k // 64, 2, 4, 8)        # r, c, b, h, i, e
    return t.permute(0, 2, 4, 3, 1, 5).contiguous().reshape(n, k)  # r, b, i, (h, c), e


def tile_weight_f16(w: torch.Tensor) -> torch.Tensor:
    """[n, k] row-major (bf16 or any float) -> DTREE_W_TILED_F16: tile_weight's
    order with fp16 elements (nearest even, saturating at +-65504; every bf16
    of magnitude 2^-17 .. 65504 converts exactly)."""
    if w.dtype != torch.float16:
        w = w.float().clamp(-65504.0, 65504.0).to(torch.float16)
    return tile_weight(w)


def fp16_exact_bf16(t: torch.Tensor) -> torch.Tensor:
    """bf16 weights that fp16 holds exactly: magnitudes below 2^-17 (3e-4 of
    an N(0, 0.02) draw) become zero; every other bf16 up to 65504 converts to
    fp16 without rounding, so the bf16 model and its DTREE_W_TILED_F16 copy
    are the same matrix."""
    t = t.to(torch.bfloat16)
    return torch.where(t.abs() < 2.0 ** -17, torch.zeros_like(t), t)


def untile_weight(t: torch.Tensor) -> torch.Tensor:
    """Inverse permutation of tile_weight / tile_weight_f16 (element type kept)."""
    n, k = t.shape
    u = t.reshape(n // 32, k // 64, 4, 2, 32, 8)         # r, b, i, h, c, e
    return u.permute(0, 4, 1, 3, 2, 5).contiguous().reshape(n, k)


def tiled_rows(t: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """Rows of a tiled [n, k] matrix in row-major order (embedding lookups)."""
    n, k = t.shape
    v = t.reshape(n // 32, k // 64, 4, 2, 32, 8)
    r = rows.long().reshape(-1)
    g = v[r // 32, :, :, :, r % 32, :]                    # [R, b, i, h, e]
    return g.permute(0, 1, 3, 2, 4).reshape(*rows.shape, k)


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    F, H = gate.shape
    if F % 16:
        raise ValueError("intermediate size must be a multiple of 16")
    return torch.stack([gate.reshape(F // 16, 16, H), up.reshape(F // 16, 16, H)], dim=1).reshape(2 * F, H)


def split_gate_up(wgu: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    F2, H = wgu.shape
    v = wgu.reshape(F2 // 32, 2, 16, H)
    return v[:, 0].reshape(F2 // 2, H), v[:, 1].reshape(F2 // 2, H)


def q4_to_tiled(wq: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """MLX quantized layout -> DTREE_W_Q4G64.

    In: wq [N, K/8] (uint32 bit patterns in an int32 tensor; element k of a row
    is nibble k % 8 of word k // 8), scales / biases bf16 [N, K/64].
    Out: words int32 [N/32, K/64, 64, 4] -- word (l, i) of block (r, b) holds
    row 32r + l % 32, columns 64b + 32 (l // 32) + 8i + e, even e in bits
    4 (e // 2), odd e in bits 16 + 4 (e // 2) -- and (scale, bias) bf16
    [N/32, K/64, 32, 2]."""
    n, kw = wq.shape
    k = kw * 8
    if n % 32 or k % 64:
        raise ValueError("q4 weights need n % 32 == 0 and k % 64 == 0")
    nkb = k // 64
    w = (wq.to(torch.int64) & 0xFFFFFFFF).reshape(n // 32, 32, nkb, 2, 4).permute(0, 2, 3, 1, 4)  # r, b, h, c, i
    out = torch.zeros_like(w)
    for e in range(8):
        out |= ((w >> (4 * e)) & 0xF) << ((e & 1) * 16 + 4 * (e >> 1))
    out = torch.where(out >= 2 ** 31, out - 2 ** 32, out).to(torch.int32).reshape(n // 32, nkb, 64, 4)
    sc = scales.reshape(n // 32, 32, nkb).permute(0, 2, 1)
    bi = biases.reshape(n // 32, 32, nkb).permute(0, 2, 1)
    return out.contiguous(), torch.stack([sc, bi], dim=-1).contiguous()


@dataclass
class Q4Linear:
    """A q4 group-64 linear layer in DTREE_W_Q4G64 layout (see q4_to_tiled)."""
    words: torch.Tensor   # int32 [N/32, K/64, 64, 4]
    sb: torch.Tensor      # bf16 [N/32, K/64, 32, 2] (scale, bias)

    @property
    def shape(self) -> tuple[int, int]:
        return self.words.shape[0] * 32, self.words.shape[1] * 64

    @property
    def device(self) -> torch.device:
        return self.words.device

    def numel(self) -> int:
        n, k = self.shape
        return n * k

    def nbytes(self) -> int:
        return self.words.numel() * 4 + self.sb.numel() * 2

    def to(self, device) -> "Q4Linear":
        return Q4Linear(self.words.to(device), self.sb.to(device))


def q4_random_mlx(n: int, k: int, gen: torch.Generator, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Synthetic q4 layer in MLX layout: nibbles uniform in [0, 15], scales
    |N(0, 0.02)| * 8, biases N(0, 0.01) (bf16). Returns (wq int32 [n, k/8],
    scales, biases)."""
    q = torch.randint(0, 16, (n, k // 8, 8), generator=gen, device=device, dtype=torch.int64)
    wq = (q << (4 * torch.arange(8, device=device, dtype=torch.int64))).sum(-1)
    wq = torch.where(wq >= 2 ** 31, wq - 2 ** 32, wq).to(torch.int32)
    sc = torch.empty(n, k // 64, device=device).normal_(0.0, 0.02, generator=gen).abs_().mul_(8.0)
    bi = torch.empty(n, k // 64, device=device).normal_(0.0, 0.01, generator=gen)
    return wq, sc.to(torch.bfloat16), bi.to(torch.bfloat16)


def q4_unpack_tiled(lin: Q4Linear) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """DTREE_W_Q4G64 -> (q uint8 [N, K], scales [N, K/64], biases [N, K/64]) in nn.Linear order."""
    w = lin.words.to(torch.int64) & 0xFFFFFFFF                # r, b, l, i
    nr, nkb = w.shape[0], w.shape[1]
    nib = torch.stack([(w >> ((e & 1) * 16 + 4 * (e >> 1))) & 0xF for e in range(8)], dim=-1)  # r, b, l, i, e
    nib = nib.reshape(nr, nkb, 2, 32, 4, 8).permute(0, 3, 1, 2, 4, 5)  # r, c, b, h, i, e
    q = nib.reshape(nr * 32, nkb * 64).to(torch.uint8)
    sb = lin.sb.permute(0, 2, 1, 3).reshape(nr * 32, nkb, 2)
    return q, sb[..., 0], sb[..., 1]


def q4_dequant(lin: Q4Linear) -> torch.Tensor:
    """float32 [N, K] = scale * q + bias per group of 64 (nn.Linear order)."""
    q, sc, bi = q4_unpack_tiled(lin)
    return q.float() * sc.float().repeat_interleave(64, dim=1) + bi.float().repeat_interleave(64, dim=1)


def q4_rows(lin: Q4Linear, ids: torch.Tensor) -> torch.Tensor:
    """Dequantised rows `ids` of a q4 matrix (embedding lookups), bf16."""
    r = ids.long().reshape(-1)
    sub = Q4Linear(lin.words[r // 32], lin.sb[r // 32])
    full = q4_dequant(sub).reshape(len(r), 32, -1)
    return full[torch.arange(len(r), device=full.device), r % 32].to(torch.bfloat16).reshape(*ids.shape, -1)


@dataclass
class LayerWeights:
    input_norm: torch.Tensor
    wqkv: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    wo: torch.Tensor
    post_norm: torch.Tensor
    wgu: torch.Tensor
    wd: torch.Tensor


@dataclass
class Qwen3Weights:
    cfg: Qwen3Config
    embed: torch.Tensor
    final_norm: torch.Tensor
    layers: list[LayerWeights] = field(default_factory=list)
    layout: int = W_TILED
    quant: str = "bf16"   # "bf16" or "q4" (every linear and the embedding, group 64)

    @property
    def device(self) -> torch.device:
        return self.embed.device

    @classmethod
    def random_q4(cls, cfg: Qwen3Config, seed: int = 0, device="cuda", norm_jitter: float = 0.0) -> "Qwen3Weights":
        """Seeded q4 group-64 model (every linear layer and the tied embedding,
        as quantize_model quantises them): nibbles uniform in [0, 15], scales
        |N(0, 0.02)| * 8, biases N(0, 0.01). Activations stay tiled bf16."""
        cfg.validate()
        dev = torch.device(device)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)

        def q4(rows, cols):
            return Q4Linear(*q4_to_tiled(*q4_random_mlx(rows, cols, gen, dev)))

        def norm(n):
            if norm_jitter == 0.0:
                return torch.ones(n, dtype=torch.bfloat16, device=dev)
            t = torch.empty(n, dtype=torch.float32, device=dev).normal_(0.0, norm_jitter, generator=gen)
            return (1.0 + t).to(torch.bfloat16)

        H, F, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        embed = q4(cfg.vocab_size, H)
        layers = []
        for _ in range(cfg.num_hidden_layers):
            wqkv = q4(cfg.qkv_dim, H)
            wo = q4(H, cfg.q_dim)
            gq, gs, gb = q4_random_mlx(F, H, gen, dev)
            uq, us, ub = q4_random_mlx(F, H, gen, dev)
            wgu = Q4Linear(*q4_to_tiled(interleave_gate_up(gq, uq), interleave_gate_up(gs, us),
                                        interleave_gate_up(gb, ub)))
            wd = q4(H, F)
            layers.append(LayerWeights(input_norm=norm(H), wqkv=wqkv, q_norm=norm(D), k_norm=norm(D), wo=wo,
                                       post_norm=norm(H), wgu=wgu, wd=wd))
        return cls(cfg=cfg, embed=embed, final_norm=norm(H), layers=layers, layout=W_TILED, quant="q4")

    @classmethod
    def random(cls, cfg: Qwen3Config, seed: int = 0, device="cuda", std: float = 0.02,
               norm_jitter: float = 0.0, layout: int = W_TILED_F16) -> "Qwen3Weights":
        """Seeded random init on `device` (norm weights 1, or 1 + N(0, jitter));
        linear weights N(0, std) as fp16-exact bf16 (fp16_exact_bf16), stored
        in `layout` (the fp16 tiled copy by default)."""
        lay = {W_TILED_F16: tile_weight_f16, W_TILED: tile_weight}.get(layout, lambda t: t)
        cfg.validate()
        dev = torch.device(device)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)

        def lin(rows, cols):
            t = torch.empty(rows, cols, dtype=torch.float32, device=dev)
            t.normal_(0.0, std, generator=gen)
            return fp16_exact_bf16(t)

        def norm(n):
            if norm_jitter == 0.0:
                return torch.ones(n, dtype=torch.bfloat16, device=dev)
            t = torch.empty(n, dtype=torch.float32, device=dev).normal_(0.0, norm_jitter, generator=gen)
            return (1.0 + t).to(torch.bfloat16)

        H, F, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        embed = lay(lin(cfg.vocab_size, H))
        layers = []
        for _ in range(cfg.num_hidden_layers):
            wqkv = lay(lin(cfg.qkv_dim, H))
            wo = lay(lin(H, cfg.q_dim))
            gate = lin(F, H)
            up = lin(F, H)
            wd = lay(lin(H, F))
            layers.append(LayerWeights(
                input_norm=norm(H), wqkv=wqkv, q_norm=norm(D), k_norm=norm(D), wo=wo,
                post_norm=norm(H), wgu=lay(interleave_gate_up(gate, up)), wd=wd))
            del gate, up
        return cls(cfg=cfg, embed=embed, final_norm=norm(H), layers=layers, layout=layout)

    def to(self, device) -> "Qwen3Weights":
        mv = lambda t: t.to(device)  # noqa: E731
        return Qwen3Weights(
            cfg=self.cfg, embed=mv(self.embed), final_norm=mv(self.final_norm),
            layers=[LayerWeights(**{k: mv(getattr(lw, k)) for k in LayerWeights.__dataclass_fields__})
                    for lw in self.layers], layout=self.layout, quant=self.quant)

    def rowmajor(self, t) -> torch.Tensor:
        """nn.Linear-order bf16 (or, for q4, dequantised fp32) matrix."""
        if isinstance(t, Q4Linear):
            return q4_dequant(t)
        if self.layout == W_TILED_F16:  # exact: the weights are fp16_exact_bf16
            return untile_weight(t).to(torch.bfloat16)
        return untile_weight(t) if self.layout == W_TILED else t

    def embed_rows(self, ids: torch.Tensor) -> torch.Tensor:
        if isinstance(self.embed, Q4Linear):
            return q4_rows(self.embed, ids)
        if self.layout in (W_TILED, W_TILED_F16):
            return tiled_rows(self.embed, ids).to(torch.bfloat16)
        return self.embed[ids.long()]

    def nbytes_linear(self) -> int:
        if self.quant == "q4":
            return sum(lw.wqkv.nbytes() + lw.wo.nbytes() + lw.wgu.nbytes() + lw.wd.nbytes() for lw in self.layers)
        return sum(lw.wqkv.numel() + lw.wo.numel() + lw.wgu.numel() + lw.wd.numel()
                   for lw in self.layers) * 2

    def host_accessor(self):
        """(layer, name) -> numpy bf16 bits, in nn.Linear layout, for a CPU checker."""
        cfg = self.cfg
        cache: dict = {}

        def bits(t: torch.Tensor) -> np.ndarray:
            if t.dtype == torch.float32:  # dequantised q4: handed over as fp32
                return t.detach().to("cpu").contiguous().numpy()
            if t.dtype == torch.float16:  # a DTREE_W_TILED_F16 weight: exact in bf16 (fp16_exact_bf16)
                t = t.to(torch.bfloat16)
            return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)

        def lin_bits(t: torch.Tensor) -> np.ndarray:
            return bits(self.rowmajor(t))

        def get(layer, name):
            key = (layer, name)
            if key in cache:
                return cache[key]
            if layer is None:
                out = lin_bits(self.embed) if name == "embed" else bits(self.final_norm)
                if name == "embed":
                    cache[key] = out
                return out
            lw = self.layers[layer]
            q, kv = cfg.q_dim, cfg.kv_dim
            if name in ("q", "k", "v"):
                lo = {"q": 0, "k": q, "v": q + kv}[name]
                hi = lo + (q if name == "q" else kv)
                return bits(self.rowmajor(lw.wqkv)[lo:hi])
            if name in ("gate", "up"):
                g, u = split_gate_up(self.rowmajor(lw.wgu))
                return bits(g if name == "gate" else u)
            if name in ("o", "down"):
                return lin_bits(lw.wo if name == "o" else lw.wd)
            return bits({"input_norm": lw.input_norm, "q_norm": lw.q_norm, "k_norm": lw.k_norm,
                         "post_norm": lw.post_norm}[name])

        return get


@dataclass
class GdnLayerWeights:
    """One GatedDeltaNet layer (custom_qwen35_model.py:777-823 parameters).

    w_in [in_proj_dim, H]: rows in_proj_qkv (conv_dim) | in_proj_z (value_dim)
    | in_proj_b (Hv) | in_proj_a (Hv) | zero padding; conv_w fp32 [K, conv_dim]
    (conv1d.weight[:, :, 0].T, newest tap last); A_log, dt_bias fp32 [Hv];
    gnorm bf16 [Dv] (RMSNormGated weight); w_out [H, value_dim]."""
    input_norm: torch.Tensor
    w_in: torch.Tensor
    conv_w: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    gnorm: torch.Tensor
    w_out: torch.Tensor
    post_norm: torch.Tensor
    wgu: torch.Tensor
    wd: torch.Tensor


def _move(t, device):
    return t.to(device)


@dataclass
class Qwen35Weights:
    """Qwen3.5 hybrid weights: ``layers[i]`` is a GdnLayerWeights for
    GatedDeltaNet layers and a LayerWeights for the gated attention layers
    (wqkv rows: q_proj with [q | gate] per head, then k_proj, v_proj)."""
    cfg: "Qwen35Config"
    embed: torch.Tensor
    final_norm: torch.Tensor
    layers: list = field(default_factory=list)
    layout: int = W_TILED
    quant: str = "bf16"

    @property
    def device(self) -> torch.device:
        return self.final_norm.device

    @classmethod
    def random(cls, cfg, seed: int = 0, device="cuda", std: float = 0.02, norm_jitter: float = 0.0,
               quant: str = "bf16") -> "Qwen35Weights":
        """Seeded random init: linear / embedding weights N(0, std) in bf16 (or
        q4 group-64: nibbles uniform, scales |N(0, 0.02)| * 8, biases
        N(0, 0.01)); norm weights 1 (+ N(0, jitter)); conv weights U(-0.5, 0.5)
        rounded to bf16; A = U(1, 16), A_log = log A; dt_bias 1 (the init of
        custom_qwen35_model.py:812-815 with A bounded away from 0)."""
        from .config import Qwen35Config  # noqa: F401  (type of cfg)
        cfg.validate()
        if quant not in ("bf16", "q4"):
            raise ValueError("quant must be 'bf16' or 'q4'")
        dev = torch.device(device)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        H, F = cfg.hidden_size, cfg.intermediate_size

        def lin_bf16(rows, cols):
            t = torch.empty(rows, cols, dtype=torch.float32, device=dev)
            t.normal_(0.0, std, generator=gen)
            return fp16_exact_bf16(t)

        def pad_rows(t, rows):
            return torch.cat([t, t.new_zeros(rows - t.shape[0], *t.shape[1:])]) if rows > t.shape[0] else t

        def lin(rows, cols, pad_to=None):
            if quant == "q4":
                wq, s, b = q4_random_mlx(rows, cols, gen, dev)
                if pad_to:
                    wq, s, b = pad_rows(wq, pad_to), pad_rows(s, pad_to), pad_rows(b, pad_to)
                return Q4Linear(*q4_to_tiled(wq, s, b))
            t = lin_bf16(rows, cols)
            return tile_weight_f16(pad_rows(t, pad_to) if pad_to else t)

        def gate_up():
            if quant == "q4":
                gq, gs, gb = q4_random_mlx(F, H, gen, dev)
                uq, us, ub = q4_random_mlx(F, H, gen, dev)
                return Q4Linear(*q4_to_tiled(interleave_gate_up(gq, uq), interleave_gate_up(gs, us),
                                            interleave_gate_up(gb, ub)))
            return tile_weight_f16(interleave_gate_up(lin_bf16(F, H), lin_bf16(F, H)))

        def norm(n):
            if norm_jitter == 0.0:
                return torch.ones(n, dtype=torch.bfloat16, device=dev)
            t = torch.empty(n, dtype=torch.float32, device=dev).normal_(0.0, norm_jitter, generator=gen)
            return (1.0 + t).to(torch.bfloat16)

        embed = lin(cfg.vocab_size, H)
        layers = []
        for i in range(cfg.num_hidden_layers):
            if cfg.is_linear(i):
                Hv = cfg.linear_num_value_heads
                in_rows = cfg.conv_dim + cfg.value_dim + 2 * Hv
                conv = torch.empty(cfg.linear_conv_kernel_dim, cfg.conv_dim, device=dev).uniform_(-0.5, 0.5,
                                                                                                  generator=gen)
                A = torch.empty(Hv, device=dev).uniform_(1.0, 16.0, generator=gen)
                layers.append(GdnLayerWeights(
                    input_norm=norm(H), w_in=lin(in_rows, H, pad_to=cfg.in_proj_dim),
                    conv_w=conv.to(torch.bfloat16).float(), A_log=torch.log(A), dt_bias=torch.ones(Hv, device=dev),
                    gnorm=norm(cfg.linear_value_head_dim), w_out=lin(H, cfg.value_dim), post_norm=norm(H),
                    wgu=gate_up(), wd=lin(H, F)))
            else:
                layers.append(LayerWeights(
                    input_norm=norm(H), wqkv=lin(cfg.attn_qkv_dim, H), q_norm=norm(cfg.head_dim),
                    k_norm=norm(cfg.head_dim), wo=lin(H, cfg.q_dim), post_norm=norm(H), wgu=gate_up(),
                    wd=lin(H, F)))
        # bf16 weights are held as the fp16 tiled copy; q4 keeps tiled bf16
        # activations (its random residual stream leaves the fp16 range)
        return cls(cfg=cfg, embed=embed, final_norm=norm(H), layers=layers,
                   layout=W_TILED_F16 if quant == "bf16" else W_TILED, quant=quant)

    def rowmajor(self, t) -> torch.Tensor:
        if isinstance(t, Q4Linear):
            return q4_dequant(t)
        if self.layout == W_TILED_F16:
            return untile_weight(t).to(torch.bfloat16)
        return untile_weight(t) if self.layout == W_TILED else t

    def embed_rows(self, ids: torch.Tensor) -> torch.Tensor:
        if isinstance(self.embed, Q4Linear):
            return q4_rows(self.embed, ids)
        return tiled_rows(self.embed, ids).to(torch.bfloat16)

    def nbytes_linear(self) -> int:
        def nb(t):
            return t.nbytes() if isinstance(t, Q4Linear) else t.numel() * 2
        total = 0
        for lw in self.layers:
            if isinstance(lw, GdnLayerWeights):
                total += nb(lw.w_in) + nb(lw.w_out) + nb(lw.wgu) + nb(lw.wd)
            else:
                total += nb(lw.wqkv) + nb(lw.wo) + nb(lw.wgu) + nb(lw.wd)
        return total

    def host_accessor(self):
        """(layer, name) -> numpy bf16 bits / fp32 arrays in nn.Linear layout,
        with the names of oracle.qwen35.OracleQwen35."""
        cfg = self.cfg
        cache: dict = {}

        def bits(t: torch.Tensor) -> np.ndarray:
            if t.dtype == torch.float32:
                return t.detach().to("cpu").contiguous().numpy()
            if t.dtype == torch.float16:  # a DTREE_W_TILED_F16 weight: exact in bf16 (fp16_exact_bf16)
                t = t.to(torch.bfloat16)
            return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)

        def get(layer, name):
            key = (layer, name)
            if key in cache:
                return cache[key]
            if layer is None:
                out = bits(self.rowmajor(self.embed)) if name == "embed" else bits(self.final_norm)
                cache[key] = out
                return out
            lw = self.layers[layer]
            if name in ("gate", "up"):
                g, u = split_gate_up(self.rowmajor(lw.wgu))
                return bits(g if name == "gate" else u)
            if name == "down":
                return bits(self.rowmajor(lw.wd))
            if name in ("input_norm", "post_norm"):
                return bits(getattr(lw, name))
            if isinstance(lw, GdnLayerWeights):
                C, V, Hv = cfg.conv_dim, cfg.value_dim, cfg.linear_num_value_heads
                if name in ("in_qkv", "in_z", "in_b", "in_a"):
                    lo = {"in_qkv": 0, "in_z": C, "in_b": C + V, "in_a": C + V + Hv}[name]
                    n = {"in_qkv": C, "in_z": V, "in_b": Hv, "in_a": Hv}[name]
                    return bits(self.rowmajor(lw.w_in)[lo:lo + n])
                if name == "out":
                    return bits(self.rowmajor(lw.w_out))
                t = {"conv": lw.conv_w, "A_log": lw.A_log, "dt_bias": lw.dt_bias, "gnorm": lw.gnorm}[name]
                return bits(t)
            q2, kv = 2 * cfg.q_dim, cfg.num_key_value_heads * cfg.head_dim
            if name in ("q", "k", "v"):
                lo = {"q": 0, "k": q2, "v": q2 + kv}[name]
                return bits(self.rowmajor(lw.wqkv)[lo:lo + (q2 if name == "q" else kv)])
            if name == "o":
                return bits(self.rowmajor(lw.wo))
            return bits({"q_norm": lw.q_norm, "k_norm": lw.k_norm}[name])

        return get
