"""Seeded synthetic inputs for the benchmark configurations (no checkpoint is needed or available).

Distributions (one per configuration of the benchmark definition):
  int4 weights  codes uniform in 0..15, packed two per byte (low nibble = even column);
                scale fp16 ~ U[1e-3, 2e-2] per (row, 128-column group); min fp16 = -7.5*scale + N(0,1)*scale
  int8 head     codes int8 uniform in [-127, 127]; per-row scale fp16 ~ U[1e-3, 1e-2]
  activations   fp16 ~ N(0, 1)
  LayerNorm w   fp16 ~ U[0.5, 1.5] per layer (the benchmark leaves them unspecified; not 1, so tests see their index)
Draw order inside one generator: codes, scale, min jitter (then x when asked for). A CPU torch.Generator makes the
values identical on every host; `device="cuda"` draws on the GPU instead (fast, for benchmarks whose values do not
matter, not bit-identical to the CPU draw).
"""
import torch

G = 128


def generator(seed: int, device="cpu") -> torch.Generator:
    return torch.Generator(device=device).manual_seed(int(seed))


def int4_weights(N: int, K: int, gen: torch.Generator, device="cpu"):
    """(q uint8 [N, K/2], scale fp16 [N, K/128], min fp16 [N, K/128]) drawn from `gen`."""
    dev = gen.device
    codes = torch.randint(0, 16, (N, K), generator=gen, device=dev, dtype=torch.uint8)
    q = (codes[:, 0::2] | (codes[:, 1::2] << 4)).contiguous()
    del codes
    s = (torch.rand(N, K // G, generator=gen, device=dev) * (2e-2 - 1e-3) + 1e-3).half()
    jitter = torch.randn(N, K // G, generator=gen, device=dev)
    m = (-7.5 * s.float() + jitter * s.float()).half()
    return q.to(device), s.contiguous().to(device), m.contiguous().to(device)


def int8_weights(N: int, K: int, gen: torch.Generator, device="cpu"):
    """(codes int8 [N, K] in [-127, 127], scale fp16 [N])."""
    dev = gen.device
    q = torch.randint(-127, 128, (N, K), generator=gen, device=dev, dtype=torch.int8)
    s = (torch.rand(N, generator=gen, device=dev) * (1e-2 - 1e-3) + 1e-3).half()
    return q.to(device), s.to(device)


def ln_weights(H: int, gen: torch.Generator, device="cpu"):
    """LayerNorm weights fp16 [H] ~ U[0.5, 1.5]."""
    return (torch.rand(H, generator=gen, device=gen.device) + 0.5).half().to(device)


def activations(shape, gen: torch.Generator, device="cpu", dtype=torch.float16):
    return torch.randn(shape, generator=gen, device=gen.device).to(dtype).to(device)


def gemv_case(N: int, K: int, seed: int, device="cpu"):
    """One int4 GEMV problem: (x fp16 [K], q, s, m)."""
    g = generator(seed)
    q, s, m = int4_weights(N, K, g)
    x = activations(K, g)
    return x.to(device), q.to(device), s.to(device), m.to(device)


def int8_case(N: int, K: int, seed: int, device="cpu"):
    """One int8 head problem: (x fp16 [K], codes int8 [N, K], scale fp16 [N])."""
    g = generator(seed)
    q, s = int8_weights(N, K, g)
    x = activations(K, g)
    return x.to(device), q.to(device), s.to(device)


def prefill_case(M: int, N: int, K: int, seed: int, device="cpu"):
    """One prefill problem: (X fp16 [M, K], q, s, m)."""
    g = generator(seed)
    q, s, m = int4_weights(N, K, g)
    X = activations((M, K), g)
    return X.to(device), q.to(device), s.to(device), m.to(device)
