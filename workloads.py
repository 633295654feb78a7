"""Synthetic inputs of the five BASELINE.json configurations (shared by bench.py and tests).

Each builder draws seeded tensors on ``device`` (weights from seed 0, activations from
seed 1, as the configurations are stated) and returns the checkpoint-form operands the
FP8 linear methods load: e4m3 ``[N, K]`` weights plus the recipe's weight scales.

* Cfg1 per-tensor (Qwen3-0.6B MLP): W ~ N(0, 0.02) [3072, 1024], one fp32 scale
  amax/448 broadcast to ``[N]`` as the loader stores it; x ~ N(0, 1).
* Cfg2 W8A16 (Llama-3-8B decode): W ~ N(0, 0.02) per-row quantized, fp32 ``[N, 1]``
  scales; x ~ N(0, 1) with 1% of the K channels (seeded choice) scaled by 20.
* Cfg3 rowwise (Qwen2-7B prefill): W per-row quantized; x as Cfg2; bias ~ N(0, 1) bf16.
* Cfg4 block-128 (DeepSeek-V3 dense): W ~ N(0, 1), each 128 x 128 block rescaled to an
  amax of 10^U(-3, 0), quantized with s = amax_blk / 448 into fp32 ``[N/128, K/128]``;
  x ~ N(0, 1).
* Cfg5 MXFP8 (Llama-3-70B MLP): W ~ N(0, 1) MX-quantized (per-32 UE8M0 codes); x rows
  ~ Student-t(df = 3).

The weight quantizers here are plain torch (they run on the device so the full-size
configurations build in seconds); they produce checkpoint data, they are not the
kernels under test.
"""

from __future__ import annotations

import math

import torch

E4M3 = torch.float8_e4m3fn

CFG1 = {"name": "cfg1_per_tensor", "shapes": [("mlp", 3072, 1024)], "ms": [1, 8]}
CFG2 = {"name": "cfg2_w8a16", "shapes": [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096),
                                         ("down", 4096, 14336)], "ms": [1, 4, 16, 32]}
CFG3 = {"name": "cfg3_rowwise", "shapes": [("gate_up", 37888, 3584), ("down", 3584, 18944)], "ms": [512, 2048, 8192]}
CFG4 = {"name": "cfg4_block128", "shapes": [("up", 18432, 7168), ("down", 7168, 18432)], "ms": [1, 32, 256, 4096]}
CFG5 = {"name": "cfg5_mxfp8", "shapes": [("gate_up", 57344, 8192), ("down", 8192, 28672)], "ms": [1, 64, 512, 2048]}
CONFIGS = [CFG1, CFG2, CFG3, CFG4, CFG5]


def _gen(device, seed: int) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


def quant_rows(wf: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-row e4m3 quant: ``s[n] = amax(W[n]) / 448`` (fp32)."""
    s = wf.abs().amax(dim=1).clamp_min(1e-12) / 448.0
    return (wf / s[:, None]).clamp(-448, 448).to(E4M3), s.float()


def quant_tensor(wf: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """One fp32 scale ``amax(W) / 448`` for the whole tensor."""
    s = wf.abs().amax().clamp_min(1e-12) / 448.0
    return (wf / s).clamp(-448, 448).to(E4M3), s.float()


def quant_blocks(wf: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """128 x 128 block e4m3 quant (N, K multiples of 128): fp32 ``[N/128, K/128]``."""
    n, k = wf.shape
    blocks = wf.reshape(n // 128, 128, k // 128, 128)
    s = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-12) / 448.0
    q = (blocks / s[:, None, :, None]).clamp(-448, 448).reshape(n, k).to(E4M3)
    return q, s.float()


def quant_mx(wf: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-32 MX quant with UE8M0 codes: e = ceil(log2(amax / 448)) (clamped to
    [-126, 127]), code = e + 127 (0 for an all-zero group), q = x / 2^e."""
    n, k = wf.shape
    g = wf.float().reshape(n, k // 32, 32)
    amax = g.abs().amax(dim=-1)
    e = torch.ceil(torch.log2((amax / 448.0).clamp_min(1e-38))).clamp(-126, 127)
    zero = amax == 0
    code = torch.where(zero, torch.zeros_like(e), e + 127).to(torch.uint8)
    q = (g / torch.exp2(torch.where(zero, torch.zeros_like(e), e))[..., None]).clamp(-448, 448)
    return q.reshape(n, k).to(E4M3), code


def outlier_activations(m: int, k: int, device, seed: int = 1, dtype=torch.bfloat16) -> torch.Tensor:
    """x ~ N(0, 1) with 1% of the K channels (one seeded choice for all rows) x20."""
    g = _gen(device, seed)
    x = torch.randn(m, k, generator=g, device=device)
    idx = torch.randperm(k, generator=g, device=device)[: max(1, k // 100)]
    x[:, idx] *= 20.0
    return x.to(dtype)


def normal_activations(m: int, k: int, device, seed: int = 1, dtype=torch.bfloat16) -> torch.Tensor:
    return torch.randn(m, k, generator=_gen(device, seed), device=device).to(dtype)


def student_t_activations(m: int, k: int, device, seed: int = 1, dtype=torch.bfloat16) -> torch.Tensor:
    """Rows of Student-t(df = 3) draws: z / sqrt(chi2_3 / 3) from seeded normals."""
    g = _gen(device, seed)
    z = torch.randn(m, k, generator=g, device=device)
    chi = torch.randn(3, m, k, generator=g, device=device).square().sum(dim=0)
    return (z / torch.sqrt(chi / 3.0)).to(dtype)


def cfg1_weights(n: int, k: int, device, seed: int = 0):
    wf = torch.randn(n, k, generator=_gen(device, seed), device=device) * 0.02
    q, s = quant_tensor(wf)
    return q, s.expand(n).contiguous()


def cfg23_weights(n: int, k: int, device, seed: int = 0):
    wf = torch.randn(n, k, generator=_gen(device, seed), device=device) * 0.02
    return quant_rows(wf)


def cfg4_weights(n: int, k: int, device, seed: int = 0):
    g = _gen(device, seed)
    wf = torch.randn(n, k, generator=g, device=device)
    nb, kb = n // 128, k // 128
    target = torch.pow(10.0, -3.0 * torch.rand(nb, kb, generator=g, device=device))
    blocks = wf.reshape(nb, 128, kb, 128)
    amax = blocks.abs().amax(dim=(1, 3))
    blocks.mul_((target / amax)[:, None, :, None])
    return quant_blocks(wf)


def cfg5_weights(n: int, k: int, device, seed: int = 0):
    wf = torch.randn(n, k, generator=_gen(device, seed), device=device)
    return quant_mx(wf)


def bias_vector(n: int, device, seed: int = 2, dtype=torch.bfloat16) -> torch.Tensor:
    return torch.randn(n, generator=_gen(device, seed), device=device).to(dtype)


def gemm_flops(m: int, n: int, k: int) -> float:
    return 2.0 * m * n * k


def sample_rows(m: int, tile: int = 128, seed: int = 3) -> torch.Tensor:
    """Row indices for a sampled check: every row up to 64; beyond, the first and last
    8 rows plus two seeded rows of every ``tile``-row tile (so each M tile is seen)."""
    if m <= 64:
        return torch.arange(m)
    g = torch.Generator().manual_seed(seed)
    picks = [torch.arange(8), torch.arange(m - 8, m)]
    for t0 in range(0, m, tile):
        size = min(tile, m - t0)
        picks.append(t0 + torch.randperm(size, generator=g)[: min(2, size)])
    return torch.unique(torch.cat(picks))


def mx_code_bytes(n: int, k: int) -> int:
    return n * math.ceil(k / 32)
