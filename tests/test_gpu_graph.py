"""Capture safety: a decode-layer sequence of the fused ops, a decode tail (gates, paged append,
samplers) and a prefill layer's fused rotations (matrix-core transforms, per-launch dynamic LDS) are
each captured in a HIP graph (through torch.cuda.CUDAGraph on its capture stream) and replayed several
times with new device-side inputs between replays; every replay must equal the eager run on the same
inputs bit for bit.  The ops allocate nothing, synchronise nothing and record no memset."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import dev_normal

pytestmark = pytest.mark.gpu


def layer(buf):
    ffi.rms_norm_res_in(buf["a_out"], buf["w1"], buf["y"], buf["resid"], 1e-6)
    ffi.rope(buf["q"], buf["q"], buf["k"], buf["k"], buf["inv"], 0, buf["pos"], buf["qn"], buf["kn"], 1e-6, 0.0,
             exl3r.ROPE_NEOX, 1.0)
    ffi.silu_mul(buf["gate"], buf["up"], buf["act"])
    ffi.embedding(buf["table"], buf["ids"], buf["emb"])


def make(seed):
    f16 = torch.float16
    T, H, I, hq, hk, hd = 16, 1024, 2048, 8, 2, 128
    return {
        "a_out": dev_normal((T, H), 0, 1, 1, seed), "resid": dev_normal((T, H), 0, 4, 1, seed + 1),
        "w1": dev_normal((H,), 1, 0.1, 1, seed + 2), "y": torch.empty((T, H), device="cuda", dtype=f16),
        "q": dev_normal((T, 1, hq, hd), 0, 1, 1, seed + 3), "k": dev_normal((T, 1, hk, hd), 0, 1, 1, seed + 4),
        "qn": dev_normal((hd,), 1, 0.1, 1, seed + 5), "kn": dev_normal((hd,), 1, 0.1, 1, seed + 6),
        "inv": torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2) / hd)).astype(np.float32)).cuda(),
        "pos": torch.zeros(T, dtype=torch.int32, device="cuda"),
        "gate": dev_normal((T, I), 0, 1, 2, seed + 7), "up": dev_normal((T, I), 0, 1, 2, seed + 8),
        "act": torch.empty((T, I), device="cuda", dtype=torch.bfloat16),
        "table": dev_normal((500, H), 0, 0.02, 2, seed + 9), "ids": torch.zeros(T, dtype=torch.int64, device="cuda"),
        "emb": torch.empty((T, H), device="cuda", dtype=torch.float32),
    }


def test_graph_replays_match_eager():
    g_buf = make(0)
    e_buf = {k: v.clone() for k, v in g_buf.items()}
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        layer(g_buf)                     # warm-up outside capture (first-launch setup)
    torch.cuda.synchronize()
    for k in g_buf:                      # restart both copies from identical state
        g_buf[k].copy_(e_buf[k])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer(g_buf)
    torch.cuda.synchronize()
    rng = np.random.default_rng(1)
    for rep in range(4):
        pos = torch.from_numpy(rng.integers(0, 40000, 16).astype(np.int32))
        ids = torch.from_numpy(rng.integers(0, 500, 16).astype(np.int64))
        for b in (g_buf, e_buf):
            b["pos"].copy_(pos)
            b["ids"].copy_(ids)
            b["a_out"].copy_(dev_normal((16, 1024), 0, 1, 1, 100 + rep))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        layer(e_buf)
        torch.cuda.synchronize()
        for k in ("resid", "y", "q", "k", "act", "emb"):
            assert torch.equal(g_buf[k].view(torch.uint8) if g_buf[k].dtype != torch.float32 else g_buf[k],
                               e_buf[k].view(torch.uint8) if e_buf[k].dtype != torch.float32 else e_buf[k]), (rep, k)


def test_ops_on_side_stream():
    buf = make(3)
    ref = {k: v.clone() for k, v in buf.items()}
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        layer(buf)
    s.synchronize()
    layer(ref)
    torch.cuda.synchronize()
    for k in ("resid", "y", "q", "k", "act", "emb"):
        assert torch.equal(buf[k], ref[k]), k


def tail(buf):
    """The attention-output gate, the paged append and the sampling step of a decode iteration."""
    ffi.deinterleave_qg(buf["qg"], buf["qd"], buf["gd"], 64)
    ffi.rope_paged_kv(buf["qd"], buf["qd"], buf["kk"], buf["kk"], buf["vv"], buf["inv"], 0, buf["sl"], None, None,
                      1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, buf["kc"], buf["vc"], buf["bt"], buf["sl"])
    ffi.mul_sigmoid_(buf["att"], buf["gd"])
    ffi.gated_rms_norm(buf["att"], buf["gw"], buf["gy"], buf["gd"], 1e-6, 0.0, 1, False, 1)
    ffi.argmax_sample(buf["logits"], buf["ids_a"], 30001)
    ffi.gumbel_sample(buf["logits"], buf["ids_g"], 0, 4242)
    ffi.gumbel_noise(buf["logits"], buf["noisy"], 4243)


def make_tail(seed):
    T, heads, hd, hk, V = 16, 4, 64, 2, 32000
    f16 = torch.float16
    return {
        "qg": dev_normal((T, heads * 2 * hd), 0, 1, 1, seed),
        "qd": torch.empty((T, 1, heads, hd), device="cuda", dtype=f16),
        "gd": torch.empty((T, heads * hd), device="cuda", dtype=f16),
        "kk": dev_normal((T, 1, hk, hd), 0, 1, 1, seed + 1), "vv": dev_normal((T, 1, hk, hd), 0, 1, 1, seed + 2),
        "inv": torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2) / hd)).astype(np.float32)).cuda(),
        "kc": torch.zeros((40, 16, hk, hd), device="cuda", dtype=f16),
        "vc": torch.zeros((40, 16, hk, hd), device="cuda", dtype=f16),
        "bt": torch.arange(T * 2, dtype=torch.int32, device="cuda").view(T, 2),
        "sl": torch.zeros(T, dtype=torch.int32, device="cuda"),
        "att": dev_normal((T, heads * hd), 0, 1, 1, seed + 3),
        "gw": dev_normal((heads * hd,), 1, 0.1, 0, seed + 4),
        "gy": torch.empty((T, heads * hd), device="cuda", dtype=f16),
        "logits": dev_normal((T, V), 0, 3, 2, seed + 5),
        "ids_a": torch.zeros(T, dtype=torch.int64, device="cuda"),
        "ids_g": torch.zeros(T, dtype=torch.int64, device="cuda"),
        "noisy": torch.empty((T, V), device="cuda", dtype=torch.float32),
    }


def test_tail_graph_replays_match_eager():
    """Gated ops, the fused paged append and both samplers under capture: each replay, with new
    logits, projections and cache lengths written between replays, equals the eager run bitwise (the
    argmax's clear / convert launches are kernels, not memsets, so replays start from a clean slot)."""
    g_buf = make_tail(20)
    e_buf = {k: v.clone() for k, v in g_buf.items()}
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        tail(g_buf)
    torch.cuda.synchronize()
    for k in g_buf:
        g_buf[k].copy_(e_buf[k])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tail(g_buf)
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    for rep in range(4):
        sl = torch.from_numpy(rng.integers(0, 16, 16).astype(np.int32))
        for b in (g_buf, e_buf):
            b["sl"].copy_(sl)
            b["logits"].copy_(dev_normal((16, 32000), 0, 3, 2, 200 + rep))
            b["qg"].copy_(dev_normal((16, 512), 0, 1, 1, 300 + rep))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        tail(e_buf)
        torch.cuda.synchronize()
        for k in ("qd", "gd", "kk", "kc", "vc", "att", "gy", "ids_a", "ids_g", "noisy"):
            a, b = g_buf[k], e_buf[k]
            if a.dtype in (torch.float16, torch.bfloat16):
                a, b = a.view(torch.int16), b.view(torch.int16)
            assert torch.equal(a, b), (rep, k)
        assert not torch.equal(g_buf["ids_a"], torch.zeros_like(g_buf["ids_a"]))


def prefill(buf):
    """The fused rotations of a prefill layer (their matrix-core defaults): the previous projection's output
    rotation into the residual norm and three projection inputs, the q / k / v output rotations into RoPE and
    the paged append (post-scales staged in LDS), the gated norm into o_proj's input rotation, and the MLP
    tail from the raw gate / up outputs."""
    ffi.rms_norm_had(buf["x"], buf["w"], [buf["xq"], buf["xk"], buf["xv"]], [buf["sq"], buf["sk"], buf["sv"]], 1e-6,
                     r=buf["r"], rotate_x=True, x_post_scale=buf["svx"])
    ffi.rope_paged_kv_had(buf["q"], buf["oq"], buf["k"], buf["ok"], buf["v"], buf["inv"], 0, buf["sl"], buf["qn"],
                          buf["kn"], 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, buf["kc"], buf["vc"], buf["bt"], buf["sl"],
                          q_post_scale=buf["pq"], k_post_scale=buf["pk"], v_post_scale=buf["pv"])
    ffi.gated_rms_norm_had(buf["ga"], buf["gw"], buf["gg"], buf["go"], 1e-6, buf["gs"], pre_rows=4)
    ffi.act_mul_had("silu", buf["mg"], buf["mu"], buf["mo"], buf["ms"], rotate_x=True, rotate_y=True,
                    x_post_scale=buf["mpg"], y_post_scale=buf["mpu"])


def make_prefill(seed):
    T, H, hq, hk, hd, I = 384, 1024, 8, 2, 128, 2048
    f16 = torch.float16

    def sign(n, s):
        g = torch.Generator(device="cuda").manual_seed(s)
        return torch.where(torch.rand(n, generator=g, device="cuda") < 0.5, -1.0, 1.0).to(f16)

    b = {"x": dev_normal((T, H), 0, 1, 1, seed), "r": dev_normal((T, H), 0, 4, 0, seed + 1),
         "w": dev_normal((H,), 1, 0.1, 1, seed + 2), "svx": sign(H, seed + 3)}
    for i, n in enumerate(("xq", "xk", "xv")):
        b[n] = torch.empty((T, H), device="cuda", dtype=f16)
        b["s" + n[1]] = sign(H, seed + 4 + i)
    b.update({"q": dev_normal((1, T, hq, hd), 0, 2, 1, seed + 10), "k": dev_normal((1, T, hk, hd), 0, 2, 1, seed + 11),
              "v": dev_normal((1, T, hk, hd), 0, 2, 1, seed + 12),
              "oq": torch.empty((1, T, hq, hd), device="cuda", dtype=f16),
              "ok": torch.empty((1, T, hk, hd), device="cuda", dtype=f16),
              "qn": dev_normal((hd,), 1, 0.1, 1, seed + 13), "kn": dev_normal((hd,), 1, 0.1, 1, seed + 14),
              "inv": torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2) / hd)).astype(np.float32)).cuda(),
              "kc": torch.zeros((8, 64, hk, hd), device="cuda", dtype=f16),
              "vc": torch.zeros((8, 64, hk, hd), device="cuda", dtype=f16),
              "bt": torch.arange(8, dtype=torch.int32, device="cuda").view(1, 8),
              "sl": torch.zeros(1, dtype=torch.int32, device="cuda"),
              "pq": sign(hq * hd, seed + 15), "pk": sign(hk * hd, seed + 16), "pv": sign(hk * hd, seed + 17),
              "ga": dev_normal((T * 4, hd), 0, 1, 2, seed + 20), "gg": dev_normal((T * 4, hd), 0, 2, 0, seed + 21),
              "gw": dev_normal((hd,), 1, 0.1, 0, seed + 22), "go": torch.empty((T * 4, hd), device="cuda", dtype=f16),
              "gs": sign(4 * hd, seed + 23),
              "mg": dev_normal((T, I), 0, 1, 1, seed + 30), "mu": dev_normal((T, I), 0, 1, 1, seed + 31),
              "mo": torch.empty((T, I), device="cuda", dtype=f16), "ms": sign(I, seed + 32),
              "mpg": sign(I, seed + 33), "mpu": sign(I, seed + 34)})
    return b


def test_prefill_rotations_graph_replays_match_eager():
    """The matrix-core fused rotations under capture (MFMAs, dynamic LDS sized by the head count): each
    replay, with new projection outputs, residual and cache lengths written between replays, equals the
    eager run bit for bit."""
    g_buf = make_prefill(40)
    e_buf = {k: v.clone() for k, v in g_buf.items()}
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        prefill(g_buf)
    torch.cuda.synchronize()
    for k in g_buf:
        g_buf[k].copy_(e_buf[k])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        prefill(g_buf)
    torch.cuda.synchronize()
    rng = np.random.default_rng(7)
    for rep in range(4):
        sl = torch.tensor([int(rng.integers(0, 64))], dtype=torch.int32)
        new = {"x": dev_normal((384, 1024), 0, 1, 1, 400 + rep), "r": dev_normal((384, 1024), 0, 4, 0, 410 + rep),
               "q": dev_normal((1, 384, 8, 128), 0, 2, 1, 420 + rep), "mg": dev_normal((384, 2048), 0, 1, 1, 430 + rep),
               "ga": dev_normal((1536, 128), 0, 1, 2, 440 + rep)}
        for b in (g_buf, e_buf):
            b["sl"].copy_(sl)
            for k, v in new.items():
                b[k].copy_(v)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        prefill(e_buf)
        torch.cuda.synchronize()
        for k in ("r", "xq", "xk", "xv", "oq", "ok", "kc", "vc", "go", "mo"):
            a, b = g_buf[k], e_buf[k]
            if a.dtype in (torch.float16, torch.bfloat16):
                a, b = a.view(torch.int16), b.view(torch.int16)
            assert torch.equal(a, b), (rep, k)
