"""Seeded synthetic packed weights and activations (numpy), shaped like the benchmark inputs.

q4_0 / Q8_0 blocks: fp16 scale d = |N(0, 0.01)|, nibbles uniform in [0, 15] / int8 uniform in
[-127, 127]. Rows are GGUF row layout (row n = output n, K/32 consecutive blocks).
"""

import numpy as np


def q4_0_weights(rng, N, K):
    """Packed q4_0 bytes uint8 [N * K/32 * 18]."""
    nb = N * (K // 32)
    blk = np.empty((nb, 18), np.uint8)
    blk[:, 0:2] = np.abs(rng.normal(0.0, 0.01, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return blk.reshape(-1)


def q8_0_weights(rng, N, K):
    """Packed Q8_0 bytes uint8 [N * K/32 * 34]."""
    nb = N * (K // 32)
    blk = np.empty((nb, 34), np.uint8)
    blk[:, 0:2] = np.abs(rng.normal(0.0, 0.01, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    return blk.reshape(-1)


def activations(rng, shape, dtype=np.float32):
    return rng.standard_normal(shape).astype(dtype)


def exl3_tensors(rng, K, N):
    """EXL3 4-bpw tensors: random uint16 trellis [K/16, N/16, 64], suh/svh fp16 = +-|N(0, 0.01)|."""
    trellis = rng.integers(0, 65536, (K // 16, N // 16, 64), dtype=np.uint16)
    suh = (np.abs(rng.normal(0, 0.01, K)) * rng.choice([-1.0, 1.0], K)).astype(np.float16)
    svh = (np.abs(rng.normal(0, 0.01, N)) * rng.choice([-1.0, 1.0], N)).astype(np.float16)
    return trellis, suh, svh


KQ_BYTES = {12: 144, 13: 176, 14: 210, 22: 82}


def kquant_weights(rng, ty, N, K):
    """Packed Q4_K (12) / Q5_K (13) / Q6_K (14) / IQ2_S (22) bytes uint8 [N * K/256 * block]:
    uniform random quant, index, sign, scale and high-bit bytes; the fp16 fields (d and dmin;
    Q6_K and IQ2_S: d) = |N(0, 1e-4)|."""
    nb = N * (K // 256)
    sb = KQ_BYTES[ty]
    blk = rng.integers(0, 256, (nb, sb), dtype=np.uint8)
    f16 = lambda: np.abs(rng.normal(0.0, 1e-4, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if ty in (12, 13):
        blk[:, 0:2] = f16()
        blk[:, 2:4] = f16()
    elif ty == 22:
        blk[:, 0:2] = f16()
    else:
        blk[:, 208:210] = f16()
    return blk.reshape(-1)


def q4_0_weights_torch(gen, N, K, device):
    """Seeded packed q4_0 rows generated on the device (torch generator ``gen``): uint8
    [N * K/32 * 18], fp16 d = |N(0, 0.01)|, uniform nibble bytes. For workloads too large to
    build on the host (a 256-expert layer is 5.4 GB)."""
    import torch
    nb = N * (K // 32)
    blk = torch.empty((nb, 18), dtype=torch.uint8, device=device)
    d = (torch.randn(nb, generator=gen, device=device) * 0.01).abs().to(torch.float16)
    blk[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    blk[:, 2:] = torch.randint(0, 256, (nb, 16), generator=gen, device=device, dtype=torch.uint8)
    return blk.view(-1)


def q8_0_weights_torch(gen, N, K, device):
    """Seeded packed Q8_0 rows on the device: fp16 d = |N(0, 0.01)|, int8 uniform in [-127, 127]."""
    import torch
    nb = N * (K // 32)
    blk = torch.empty((nb, 34), dtype=torch.uint8, device=device)
    d = (torch.randn(nb, generator=gen, device=device) * 0.01).abs().to(torch.float16)
    blk[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    blk[:, 2:] = torch.randint(-127, 128, (nb, 32), generator=gen, device=device,
                               dtype=torch.int8).view(torch.uint8)
    return blk.view(-1)
