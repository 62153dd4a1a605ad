"""Model of the reference's f16 half-arithmetic gated activations -- TEST INFRASTRUCTURE ONLY, and
informational: it is not the checker of any exl3r kernel.

For f16 inputs the reference runs act_mul_kernel_h (kernels/activation_kernels.cuh:142-186):
  silu, _silu(half2) at :22-31:  e = hexp(-x); s = 1 + e; r = hrcp(s); a = x * r     (each op in half)
  gelu, _gelu(half) at :42-49, 61-64: a = half(float(0.5 x (1.0 + tanh_opt(c (x + 0.044715 x^3)))))
        (fp32 operands, the `1.0 +` in double, tanh_opt the hardware tanh approximation, compat.cuh:14)
  act_limit (:175-180): u clamped to [-L, L], a clamped from above, both in half;
  z = __hmul2(a, u)                                                                  (:182)
exl3r's act-mul kernels follow the reference's fp32 path instead (act_mul_kernel_f, :189-252): the
activation in fp32 and one rounding of the product, so for f16 inputs their outputs differ from the
half path.  This module measures by how much.

NVIDIA's hexp / hrcp / tanh.approx are closed intrinsics and are not reproduced: every half operation
here is modelled as correctly rounded (the exact value, or its double approximation, rounded once to
nearest even), and tanh_opt as the exact tanh.  The real half path can only be further from fp32 than
this idealised one by the intrinsics' own error."""
import numpy as np

SQRT_2_OVER_PI = 0.797884560803


def _h(v):
    """Round float64 values to f16 (nearest even; overflow to inf)."""
    with np.errstate(over="ignore"):
        return np.asarray(v, np.float64).astype(np.float16)


def act_half(act, x16):
    """The activation alone as the half path computes it: f16 in, f16 out.  act 0 = silu, 1 = gelu."""
    x = x16.astype(np.float64)
    if act == 0:
        with np.errstate(over="ignore"):
            e = _h(np.exp(-x))
        s = _h(1.0 + e.astype(np.float64))
        with np.errstate(divide="ignore"):
            r = _h(1.0 / s.astype(np.float64))
        return _h(x * r.astype(np.float64))
    xf = x.astype(np.float32).astype(np.float64)
    arg = (np.float32(SQRT_2_OVER_PI) * (xf + np.float32(0.044715) * xf * xf * xf)).astype(np.float32)
    g = (0.5 * xf * (1.0 + np.tanh(arg.astype(np.float64)))).astype(np.float32)
    return _h(g.astype(np.float64))


def act_mul_half(act, x16, y16, limit=0.0):
    """z = act(x) * y in the half path; x, y and z are float16 arrays."""
    a = act_half(act, x16)
    u = y16
    if limit != 0.0:
        lim = np.float16(limit)
        u = np.minimum(np.maximum(u, -lim), lim)
        a = np.minimum(a, lim)
    return _h(a.astype(np.float64) * u.astype(np.float64))
