"""Generates the committed golden fixtures under tests/golden/ (run here, on the CPU).

The reference ships no vectors for this path (its kernels are CUDA-only and none of its tests pin
values), so the fixtures come from independent library routines evaluated in float64 on the CPU:
  - rmsnorm.npz: torch.nn.functional.rms_norm, times (w + constant_bias) * constant_scale; RES_IN
    rows take the residual sum torch computes as (x.float() + r.float()).to(r.dtype);
  - act.npz: the textbook SiLU x / (1 + e^-x) and tanh-GELU 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))
    evaluated with mpmath at 60 significant digits (torch's float64 F.gelu cancels in 1 + tanh for
    x << 0, where bf16 still resolves the result; it is kept as z_torch64 for |x| <= 4), times y,
    with act_limit clamps;
  - rope.npz: the head norm from F.rms_norm (the f16-weight path rounds n and w + cb to half and
    multiplies in half, as torch CPU half ops do), then the rotation as a complex product
    (x1 + i x2) * (cos a + i sin a) with torch.polar / view_as_complex, pairs gathered by index
    (NeoX t, t + R/2; GPT-J 2t, 2t + 1), angle = fp32(inv_freq * fp32(pos)).
Every fixture stores its inputs as raw bit patterns and the expected outputs in float64 before the
final rounding, so a test can check an implementation against RNE(expected) in ulps.

Usage: python tests/golden/make_golden.py
"""
import os

import mpmath
import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
TD = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


def bits(t):
    """torch tensor -> numpy storage (float32 or raw uint16)."""
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def gen(shape, mean, std, g):
    return torch.randn(shape, generator=g, dtype=torch.float64) * std + mean


def rmsnorm_cases(g):
    cases = []
    specs = [
        # rows, dim, xt, wt, yt, rt (None: plain), eps, cb, cs
        (6, 64, 1, 1, 1, None, 1e-6, 0.0, 1.0),
        (3, 1024, 1, 1, 1, None, 1e-6, 0.0, 1.0),
        (3, 1024, 2, 2, 2, None, 1e-6, 0.0, 1.0),
        (3, 1000, 0, 2, 1, None, 1e-5, 1.0, 1.0),
        (5, 512, 1, 1, 0, None, 1e-6, 0.0, 0.5),
        (2, 2048, 1, 1, 1, 1, 1e-6, 0.0, 1.0),
        (2, 2048, 1, 1, 1, 0, 1e-6, 0.0, 1.0),
        (2, 2048, 2, 2, 2, 2, 1e-6, 0.0, 1.0),
        (3, 136, 1, 2, 1, 0, 1e-6, 1.0, 1.0),
    ]
    for rows, dim, xt, wt, yt, rt, eps, cb, cs in specs:
        x = gen((rows, dim), 0.0, 1.0, g).to(TD[xt])
        w = gen((dim,), 1.0, 0.1, g).to(TD[wt])
        case = dict(rows=rows, dim=dim, xt=xt, wt=wt, yt=yt, rt=-1 if rt is None else rt, eps=eps, cb=cb, cs=cs,
                    x=bits(x), w=bits(w))
        xf = x.float()
        if xt == 1:
            xf = xf.clamp(-65504.0, 65504.0)
        if rt is not None:
            r = gen((rows, dim), 0.0, 4.0, g).to(TD[rt])
            h = (xf + r.float()).to(TD[rt])
            case["r"] = bits(r)
            case["h"] = bits(h)
            src = h.double()
        else:
            src = xf.double()
        wd = w.double() + cb if cb != 0.0 else w.double()
        y = F.rms_norm(src, (dim,), eps=eps) * wd * cs
        case["y64"] = y.numpy()
        cases.append(case)
    return cases


def hp_act(act, x):
    """SiLU / tanh-GELU of a float64 x at 60 significant digits, rounded to float64."""
    with mpmath.workdps(60):
        v = mpmath.mpf(x)
        if act == "silu":
            r = v / (1 + mpmath.exp(-v))
        else:
            u = mpmath.sqrt(2 / mpmath.pi) * (v + mpmath.mpf("0.044715") * v ** 3)
            r = mpmath.mpf("0.5") * v * (1 + mpmath.tanh(u))
        return float(r)


def act_cases(g):
    cases = []
    specials = torch.tensor([0.0, -0.0, 1.0, -1.0, 3.5, -3.5, 8.0, -8.0, 15.0, -15.0, 30.0, -30.0, 1e-3, -1e-3],
                            dtype=torch.float64)
    for act in ("silu", "gelu"):
        for it, zt, limit in ((1, 1, 0.0), (2, 2, 0.0), (0, 1, 0.0), (1, 1, 4.0), (2, 0, 0.0)):
            rows, cols = 4, 96
            x = gen((rows, cols), 0.0, 3.0, g)
            x.view(-1)[: specials.numel()] = specials
            y = gen((rows, cols), 0.0, 1.0, g)
            x, y = x.to(TD[it]), y.to(TD[it])
            xd, yd = x.double(), y.double()
            at = F.silu(xd) if act == "silu" else F.gelu(xd, approximate="tanh")
            a = torch.tensor([hp_act(act, float(v)) for v in xd.view(-1)], dtype=torch.float64).view(xd.shape)
            if limit != 0.0:
                yd = yd.clamp(-limit, limit)
                a = a.clamp(max=limit)
                at = at.clamp(max=limit)
            cases.append(dict(act=0 if act == "silu" else 1, it=it, zt=zt, limit=limit, rows=rows, cols=cols,
                              x=bits(x), y=bits(y), z64=(a * yd).numpy(), z_torch64=(at * yd).numpy()))
    return cases


def rope_cases(g):
    cases = []
    specs = [
        # bsz, seq, hq, hk, hd, R, mode, dt, norm (None|wt), cb, attn, pos kind
        (2, 5, 3, 2, 64, 64, 2, 1, 1, 0.0, 1.0, "scalar"),
        (2, 5, 3, 2, 64, 64, 1, 1, 1, 0.0, 1.0, "positions"),
        (1, 6, 2, 1, 128, 128, 2, 1, 2, 1.0, 1.0, "ids"),
        (1, 4, 2, 2, 128, 64, 1, 1, None, 0.0, 1.0, "ids"),
        (2, 3, 4, 2, 32, 16, 2, 2, 2, 0.0, 0.8, "positions"),
        (1, 3, 2, 1, 128, 128, 2, 1, 1, 1.0, 1.0, "scalar"),
    ]
    for bsz, seq, hq, hk, hd, R, mode, dt, nwt, cb, attn, pk in specs:
        io = TD[dt]
        q = gen((bsz, seq, hq, hd), 0.0, 1.0, g).to(io)
        k = gen((bsz, seq, hk, hd), 0.0, 1.0, g).to(io)
        theta = 1e6
        inv = (1.0 / (theta ** (torch.arange(0, R, 2, dtype=torch.float64) / R))).float()
        position = 0
        positions = None
        position_ids = None
        if pk == "scalar":
            position = 3071
            pos = torch.arange(seq, dtype=torch.int64)[None, :].expand(bsz, seq) + position
        elif pk == "positions":
            positions = torch.randint(0, 32768, (bsz,), generator=g, dtype=torch.int32)
            pos = positions.long()[:, None] + torch.arange(seq)[None, :]
        else:
            position_ids = torch.randint(0, 40000, (bsz, seq), generator=g, dtype=torch.int32)
            pos = position_ids.long()
        case = dict(bsz=bsz, seq=seq, hq=hq, hk=hk, hd=hd, R=R, mode=mode, dt=dt, nwt=-1 if nwt is None else nwt,
                    cb=cb, attn=attn, eps=1e-6, position=position, q=bits(q), k=bits(k), inv_freq=inv.numpy())
        if positions is not None:
            case["positions"] = positions.numpy()
        if position_ids is not None:
            case["position_ids"] = position_ids.numpy()
        # angles: fp32 product of fp32 inv_freq and fp32 position
        ang = (inv[None, None, :] * pos.float()[:, :, None]).double()          # [bsz, seq, R/2]
        rot = torch.polar(torch.full_like(ang, attn), ang)                       # attn * e^{i a}
        outs = []
        for name, x in (("q", q), ("k", k)):
            xd = x.double()
            if nwt is not None:
                w = gen((hd,), 1.0, 0.1, g).to(TD[nwt])
                case[name + "_norm"] = bits(w)
                n = F.rms_norm(xd, (hd,), eps=1e-6)
                if nwt == 1 and dt == 1:
                    wh = (w.half() + torch.tensor(cb).half())
                    xn = wh * n.half()
                else:
                    xn = (n * (w.double() + cb)).to(io)
                case[name + "n"] = bits(xn)          # normed head, io-rounded, before the rotation
                xd = xn.double()
            t = torch.arange(R // 2)
            i1 = t if mode == 2 else 2 * t
            i2 = t + R // 2 if mode == 2 else 2 * t + 1
            z = torch.complex(xd[..., i1], xd[..., i2]) * rot[:, :, None, :]
            out = xd.clone()
            out[..., i1] = z.real
            out[..., i2] = z.imag
            outs.append(out)
        case["q64"] = outs[0].numpy()
        case["k64"] = outs[1].numpy()
        cases.append(case)
    return cases


def save(name, cases):
    flat = {"n": np.array(len(cases))}
    for i, c in enumerate(cases):
        for key, v in c.items():
            flat[f"{i}/{key}"] = np.asarray(v)
    np.savez_compressed(os.path.join(HERE, name), **flat)


def main():
    g = torch.Generator().manual_seed(0)
    save("rmsnorm.npz", rmsnorm_cases(g))
    save("act.npz", act_cases(g))
    save("rope.npz", rope_cases(g))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
