"""Shared helpers of the GPU parity tests."""
import torch

DEV = torch.device("cuda", 0)
ACTS = ["relu", "tanh", "sigmoid", "silu", "gelu", "identity"]
OPS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def gen(seed: int):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def randn(shape, g, scale=1.0):
    return torch.randn(shape, generator=g, dtype=torch.float32) * scale


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (both moved to fp64 on the CPU)."""
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    if not (bool(torch.isfinite(got).all()) and bool(torch.isfinite(ref).all())):
        return float("inf")  # NaN must never read as agreement
    den = float(ref.abs().max())
    num = float((got - ref).abs().max())
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


def rnd(t: torch.Tensor, op: torch.dtype) -> torch.Tensor:
    """Round to the operand type and back to fp32 (emulates the loader)."""
    return t.to(op).to(torch.float32)


def to_dev(t, dtype=torch.float32):
    return t.to(device=DEV, dtype=dtype).contiguous()


def report(name, **kv):
    items = " ".join(f"{k}={v}" for k, v in kv.items())
    print(f"[case] {name} {items}", flush=True)
