"""Shared tolerance for low-precision outputs.

The stated bar is max-abs 2e-2 for bf16 / fp16 outputs and gradients.  A
result stored in a 16-bit format carries its own rounding of up to half an
ulp of its magnitude (0.0156 for a bf16 value in [4, 8)), which no kernel can
avoid, so the check is |got - ref| <= 2e-2 + ulp(ref)/2 elementwise, with ref
the fp64 oracle on the same rounded inputs.

Gradients are often far below one, where that absolute bar alone says
nothing, so the check also bounds the relative error of the whole tensor,
||got - ref||_2 / ||ref||_2 <= 1e-2 (a 16-bit output's own rounding gives
about 2e-3)."""

import torch

MANTISSA = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}


def half_ulp(ref: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    m = MANTISSA[dtype]
    a = ref.abs().clamp(min=2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - m) / 2


def assert_close_lowp(got, ref, dtype, tol=2e-2, what="", rel_norm=1e-2):
    """Assert the bar above and report the plain max-abs error beside the
    error left after removing the output format's own rounding, and the
    relative norm error."""
    from parity_report import report

    got = got.double()
    ref = ref.double()
    plain = (got - ref).abs().max().item() if got.numel() else 0.0
    excess = (got - ref).abs() - half_ulp(ref, dtype)
    worst = excess.max().item() if got.numel() else 0.0
    rn = ref.norm().item()
    rel = (got - ref).norm().item() / rn if rn > 0 else (0.0 if plain == 0 else float("inf"))
    if what:
        report(f"[err] {what}: max-abs {plain:.3e}, beyond ulp/2 {worst:.3e} (bar {tol}), "
               f"rel-norm {rel:.2e} (bar {rel_norm})")
    assert worst <= tol, f"{what}: max |err| - ulp/2 = {worst:.4g} > {tol} (max |err| {plain:.4g})"
    assert rel <= rel_norm, f"{what}: ||err|| / ||ref|| = {rel:.4g} > {rel_norm}"
