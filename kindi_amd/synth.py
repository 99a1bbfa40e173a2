"""Seeded synthetic inputs of the BASELINE configs (no model files exist offline).

Ternary weights: i.i.d. trits with P(-1) = P(+1) = 0.3, P(0) = 0.4, produced directly in the reference pack format
(bcodes [C/4, R]: byte = d0 + 3 d1 + 9 d2 + 27 d3 with d = t + 1, convert.py:49-52; dpm [C/128, R] fp16 bits)
with one scale per 128-weight group, scale = fp16(exp(N(-3, 0.3))).
q8_0 experts: int8 codes ~ U[-127, 127], one fp16 scale exp(N(-6, 0.5)) per 32, as GGUF Q8_0 rows.
Activations: N(0, 1) fp32. Router logits: N(0, 1).

The generators run on the device they are given (a torch.Generator per call, seeded), so the 27B config's 5.6 GB
of packed weights are made on the GPU; the same seed gives the same values on the same device type.
"""
import torch

CFG = {
    # config 0: one ternary linear, decode
    "c0": dict(R=6144, C=2048),
    # config 1: one 2B-class layer, decode, M in {1, 4, 8}
    "c1": dict(hidden=2048, mats=[("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048),
                                  ("gate", 6144, 2048), ("up", 6144, 2048), ("down", 2048, 6144)]),
    # config 2: prefill GEMM at 9B-class shapes, M in {512, 2048}
    "c2": dict(mats=[("gate_up", 12288, 4096), ("down", 4096, 12288)]),
    # config 3: 27B-class decode sweep: 64 layers, M in {1, 16}
    "c3": dict(layers=64, mats=[("q", 5120, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 5120),
                                ("gate", 17408, 5120), ("up", 17408, 5120), ("down", 5120, 17408)]),
    # config 4: q8_0 MoE, 128 experts top-6; up [1856 x 2688], down [2688 x 1856]; M in {1, 256}
    "c4": dict(E=128, k=6, H=2688, F=1856),
}


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def tern_pack(R, C, seed, device="cpu"):
    """(bcodes uint8 [C/4, R], dpm int16 [C/128, R] holding fp16 bits) on `device`"""
    g = _gen(seed, device)
    u = torch.rand((C // 4, R, 4), generator=g, device=device)
    d = (u >= 0.3).to(torch.uint8) + (u >= 0.7).to(torch.uint8)            # P(0) = .3, P(1) = .4, P(2) = .3
    del u
    bcodes = d[..., 0] + 3 * d[..., 1] + 9 * d[..., 2] + 27 * d[..., 3]
    del d
    s = torch.exp(torch.randn((C // 128, R), generator=g, device=device) * 0.3 - 3.0)
    dpm = s.to(torch.float16).view(torch.int16)
    return bcodes.contiguous(), dpm.contiguous()


def activations(M, C, seed, device="cpu"):
    return torch.randn((M, C), generator=_gen(seed, device), device=device, dtype=torch.float32)


def q8_rows(R, C, seed, device="cpu"):
    """GGUF Q8_0 rows uint8 [R, C/32 * 34]: codes ~ U[-127, 127], scales fp16(exp(N(-6, 0.5)))"""
    g = _gen(seed, device)
    nb = C // 32
    codes = torch.randint(-127, 128, (R, nb, 32), generator=g, device=device, dtype=torch.int16).to(torch.int8)
    s = torch.exp(torch.randn((R, nb, 1), generator=g, device=device) * 0.5 - 6.0).to(torch.float16)
    out = torch.cat([s.view(torch.uint8), codes.view(torch.uint8)], dim=2)
    return out.reshape(R, nb * 34).contiguous()


def logits(M, E, seed, device="cpu"):
    return torch.randn((M, E), generator=_gen(seed, device), device=device, dtype=torch.float32)
