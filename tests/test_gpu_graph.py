"""Capture safety: a decode-layer sequence of the fused ops captured in a HIP graph (through
torch.cuda.CUDAGraph on its capture stream) is replayed several times with new device-side
positions and residual contents between replays, and every replay must equal the eager run on the
same inputs bit for bit.  The ops allocate nothing, synchronise nothing and record no memset."""
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
