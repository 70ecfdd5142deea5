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


def delta_w_check(got_w, w0, w_ref, x0, steps, *, act, alpha, gamma, bar=1e-5):
    """fp32 bar on the weight *deltas* W_T - W_0 (a bar on W itself hides
    delta errors of several percent at alpha = 1e-4).

    Where ulp(W) quantises the deltas (few steps, small alpha), two correct
    fp32 computations round W differently now and then and their deltas
    differ by more than ``bar``; the check then asks the GPU deltas to be as
    close to the float64 truth (the oracle run in float64 from the same x0 and
    W0) as the fp32 oracle's own deltas are.  Returns ``(ok, message)``."""
    from oracle import ipc_oracle as O

    w0_64 = [w.double().cpu() for w in w0]
    d_got = [g.double().cpu() - w for g, w in zip(got_w, w0_64)]
    d_ref = [r.double().cpu() - w for r, w in zip(w_ref, w0_64)]
    err = O.global_rel_err(d_got, d_ref)
    if err <= bar:
        return True, f"dW_err={err:.3e}"
    x64 = [x.double().cpu() for x in x0]
    _x, w64_t, _e = O.run_steps(x64, w0_64, steps, act=act, alpha=alpha, gamma=gamma)
    d_true = [a - b for a, b in zip(w64_t, w0_64)]
    got_vs_true = O.global_rel_err(d_got, d_true)
    ref_vs_true = O.global_rel_err(d_ref, d_true)
    ok = got_vs_true <= max(bar, 2.0 * ref_vs_true)
    return ok, f"dW_err={err:.3e} vs f64: got={got_vs_true:.3e} fp32-oracle={ref_vs_true:.3e}"
