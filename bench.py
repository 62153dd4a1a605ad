#!/usr/bin/env python3
"""Benchmark of the MI355X fused row ops (the exl3r C ABI), one JSON line on stdout.

Metric: fused norm/act/RoPE/embed HBM GB/s + % of MI355X peak; decode-step us.

A step is one pass of the config-3 prefill row ops (residual RMSNorm [8192, 5120] + SiLU-gated mul
+ GELU-gated mul [8192, 17408], bf16 I/O, fp32 arithmetic) over inputs resident in HBM; `value` is
the step's algorithmic bytes / step time.  The line also carries every other config's per-op
figures (C1 Qwen3-0.6B ops, C2 decode residual norm, C4 paged q/k-norm + RoPE, C5 embedding gather
and gather + norm), the 64-row decode-step composite fused vs the naive unfused HIP baseline, the
roofline of the step's dominant kernel (the slowest of the three, with each kernel's own time inside the
step and its HBM traffic counted by rocprofv3 in the same run), and the CPU oracle timed on this host
as a baseline.

  python bench.py [--steps K] [--warmup W]            full run (N = 1)
  python bench.py --op silu_c3 [--steps K]            one kernel only (for rocprofv3 --pmc runs)
  python bench.py --op calib_copy                     plain 1 GiB copy (counter calibration)

Inputs are seeded synthetic data of the configs' shapes (the reference ships no datasets); each
timed loop rotates over enough buffer sets that a launch never finds its operands in the 256 MB
Infinity Cache from the previous launch.
"""
import argparse
import csv
import glob
import json
import os
import shutil
import signal
import statistics
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "exllamav3-rs_amd"))

PEAK_GBS = 8000.0            # MI355X HBM3E
# The C3 step and the kernel each of its ops launches (bf16 I/O, the shapes'
# automatic launch choice).
STEP_OPS = ["rms_c3", "silu_c3", "gelu_c3"]
STEP_KERNELS = {"rms_c3": "k_rms_norm<bf16 x, bf16 y, bf16 r, RES_IN>", "silu_c3": "k_act_mul<SILU, bf16, bf16>",
                "gelu_c3": "k_act_mul<GELU, bf16, bf16>"}
METRIC = "fused norm/act/RoPE/embed HBM GB/s + % of MI355X peak; decode-step us"
OPS = ["rms_c3", "rms_q3mix", "silu_c3", "gelu_c3", "rope_c4", "rope_c4_gptj", "gather_c5", "gather_f32_c5",
       "gather_norm_c5", "rms_c1",
       "silu_c1", "rope_c1", "gather_c1", "rms_c2", "decode_fused", "decode_naive", "rope_kv_prefill",
       "rope_kv_prefill_unfused", "rope_kv_dec", "rope_kv_dec_unfused", "gated_norm_q35", "mul_sigmoid_q35",
       "deinterleave_q35", "gated_norm_had_q35", "gated_norm_had_q35_exact", "gated_norm_had_q35_unfused", "argmax_dec", "argmax_dec_torch", "argmax_dec_ws", "argmax_prefill", "argmax_prefill_torch",
       "gumbel_dec", "gumbel_dec_torch", "gumbel_dec_ws", "gumbel_prefill", "had_c3", "had_c3_mfma", "norm_had_c3",
       "norm_had_c3_exact", "norm_had_c3_unfused", "norm_had_rot_c3", "norm_had_rot_c3_exact", "norm_had_rot_c3_unfused",
       "silu_had_c3", "silu_had_c3_exact", "silu_had_c3_unfused", "rope_had_c4", "rope_had_c4_exact", "rope_had_c4_unfused", "rope_cs_c4", "rope_cs_table_c4",
       "qg_rope_q35", "qg_rope_q35_unfused",
       "rope_kv_prefill_cs", "rope_kv_had_prefill_cs", "prefill_layer_cs",
       "rope_kv_had_prefill", "rope_kv_had_prefill_exact", "rope_kv_had_prefill_unfused", "mlp_had_c3", "mlp_had_c3_exact", "mlp_had_c3_unfused",
       "prefill_layer", "prefill_layer_unfused", "calib_copy",
       "calib_copy_cached", "c3_step"]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--op", choices=OPS, default=None,
                   help="time one kernel only (c3_step: launch the C3 step sequence, for kernel-trace runs)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter runs of the dominant kernel")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    return p.parse_args()


# ------------------------------------------------------------------------------------------------
# Workloads: each builds its buffers once and returns (launch(i), bytes_per_launch, description).

class Work:
    """One timed launch.  nbytes is the algorithmic byte count of a launch; hbm_bytes, when given, is
    the least HBM traffic that can serve it (a gather whose ids repeat reads each distinct table row
    once and serves the repeats from L2 / MALL).  Such a launch's frac_peak is taken over the traffic
    the rocprofv3 counters measured for it (the committed summary), or over hbm_bytes without one."""
    def __init__(self, name, nbytes, launch, desc, sets=1, hbm_bytes=None):
        self.name, self.nbytes, self.launch, self.desc, self.sets = name, nbytes, launch, desc, sets
        self.hbm_bytes = hbm_bytes


def gen(shape, mean, std, dtype, seed):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * std + mean).to(dtype)


def sets_for(nbytes, span=600 << 20):
    """Buffer sets so that the bytes touched between two uses of one set exceed the MALL.  Launches
    under 32 MiB (the latency-bound configs 1 and 2 and the decode layer) use one set: their
    operands are cache-resident in a real decode loop too."""
    if nbytes < 32 << 20:
        return 1
    return max(2, -(-span // max(nbytes, 1)) + 1)


def zipf_ids(n, vocab, seed, s=1.1, repeat=0.05):
    import numpy as np
    rng = np.random.default_rng(seed)
    p = np.arange(1, vocab + 1, dtype=np.float64) ** -s
    p /= p.sum()
    ids = rng.choice(vocab, size=n, p=p)
    rep = np.nonzero(rng.random(n) < repeat)[0]
    for i in rep[rep > 0]:
        ids[i] = ids[i - 1]
    return ids.astype(np.int64)


def ragged_positions(seed):
    import numpy as np
    rng = np.random.default_rng(seed)
    lens = rng.integers(64, 513, 16)
    starts = rng.integers(0, 32768, 16)
    return np.concatenate([s + np.arange(n) for s, n in zip(starts, lens)]).astype(np.int32)


def make_rms(name, rows, dim, dt, res, seed, rdt=None):
    """RMSNorm, or with `res` the residual norm (r += x in place, y = norm(r)); x, y and the weight are
    `dt`, the residual `rdt` (default `dt`; float32 is the reference's Qwen3 residual stream,
    kernels/norm.cu:403)."""
    import torch
    import exl3r.ffi as ffi
    es = 2
    rdt = rdt or dt
    res_es = torch.empty((), dtype=rdt).element_size()
    nbytes = (rows * dim * (2 * es + 2 * res_es) if res else 2 * rows * dim * es) + dim * es
    sets = sets_for(nbytes)
    bufs = []
    for k in range(sets):
        x = gen((rows, dim), 0.0, 1.0, dt, seed + 3 * k)
        r = gen((rows, dim), 0.0, 4.0, rdt, seed + 3 * k + 1) if res else None
        bufs.append((x, r, torch.empty_like(x)))
    w = gen((dim,), 1.0, 0.1, dt, seed + 99)

    def launch(i):
        x, r, y = bufs[i % sets]
        if res:
            ffi.rms_norm_res_in(x, w, y, r, 1e-6)
        else:
            ffi.rms_norm(x, w, y, 1e-6)
    kind = "residual RMSNorm" if res else "RMSNorm"
    dts = str(dt).split('.')[-1] + (f" x / {str(rdt).split('.')[-1]} residual" if res and rdt != dt else "")
    return Work(name, nbytes, launch, f"{kind} [{rows},{dim}] {dts}", sets)


def make_act(name, rows, cols, dt, act, seed):
    import torch
    import exl3r.ffi as ffi
    nbytes = 3 * rows * cols * 2
    sets = sets_for(nbytes)
    bufs = [(gen((rows, cols), 0.0, 1.0, dt, seed + 2 * k), gen((rows, cols), 0.0, 1.0, dt, seed + 2 * k + 1),
             torch.empty((rows, cols), device="cuda", dtype=dt)) for k in range(sets)]
    fn = ffi.silu_mul if act == "silu" else ffi.gelu_mul

    def launch(i):
        g, u, z = bufs[i % sets]
        fn(g, u, z)
    return Work(name, nbytes, launch, f"{act.upper()}(gate)*up [{rows},{cols}] {str(dt).split('.')[-1]}", sets)


def make_rope_had(name, pos, hq, hk, hd, fused, seed=330, exact=False):
    """C4 prefill q/k on the raw f16 projection outputs: each projection's output rotation
    had_r_128(y, y, None, svh) (src/modules.rs:231), then head-norm + NeoX RoPE, in place.  One fused
    launch (exl3r_rope_had; transforms on the matrix cores, or with exact the reference's butterfly), or
    two had_r_128 launches and exl3r_rope.  Both count the fused job's bytes (C4's RoPE bytes plus both
    svh vectors)."""
    import numpy as np
    import torch
    import exl3r
    import exl3r.ffi as ffi
    T = pos.size
    nbytes = 2 * T * (hq + hk) * hd * 2 + 4 * T + 2 * hd * 2 + (hd // 2) * 4 + (hq + hk) * hd * 2
    sets = sets_for(nbytes)
    inv = torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2, dtype=np.float64) / hd)).astype(np.float32)).cuda()
    qn, kn = gen((hd,), 1.0, 0.1, torch.float16, seed + 50), gen((hd,), 1.0, 0.1, torch.float16, seed + 51)
    qs = torch.where(torch.rand(hq * hd, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16)
    ks = torch.where(torch.rand(hk * hd, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16)
    pid = torch.from_numpy(pos).cuda().view(1, -1)
    bufs = [(gen((1, T, hq, hd), 0.0, 1.0, torch.float16, seed + 2 * k),
             gen((1, T, hk, hd), 0.0, 1.0, torch.float16, seed + 2 * k + 1)) for k in range(sets)]

    def launch(i):
        q, k = bufs[i % sets]
        if fused:
            ffi.rope_had(q, q, k, k, inv, 0, None, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, q_post_scale=qs,
                         k_post_scale=ks, position_ids=pid, exact=exact)
        else:
            ffi.had_r_128(q.view(T, hq * hd), q.view(T, hq * hd), None, qs)
            ffi.had_r_128(k.view(T, hk * hd), k.view(T, hk * hd), None, ks)
            ffi.rope(q, q, k, k, inv, 0, None, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, position_ids=pid)
    kind = ("fused, butterfly" if exact else "fused") if fused else "unfused (2 had_r_128 + rope)"
    return Work(name, nbytes, launch, f"q/k output rotation + head-norm + NeoX RoPE T={T} heads {hq}/{hk}, {kind}", sets)


def make_rope_cs(name, pos, hq, hk, hd, R, dt, seed, table_only):
    """C4 with the sin / cos of the forward pass precomputed: the per-layer RoPE reading the {cos, sin}
    table (exl3r_rope_cs: C4's q/k bytes, the norm weights and the token's table row), or the table build
    that serves every layer of the forward (exl3r_rope_cs_table: the positions and inv_freq read, the
    table written)."""
    import numpy as np
    import torch
    import exl3r
    import exl3r.ffi as ffi
    T = pos.size
    inv = torch.from_numpy((1.0 / 1e6 ** (np.arange(0, R, 2, dtype=np.float64) / R)).astype(np.float32)).cuda()
    pid = torch.from_numpy(pos).cuda().view(1, -1)
    table = ffi.rope_cs_table(1, T, inv, 0, position_ids=pid)
    if table_only:
        nbytes = 4 * T + (R // 2) * 4 + T * (R // 2) * 8
        return Work(name, nbytes, lambda i: ffi.rope_cs_table(1, T, inv, 0, position_ids=pid, out=table),
                    f"{{cos, sin}} table of T={T} ragged positions, rotary {R}")
    nbytes = 2 * T * (hq + hk) * hd * 2 + T * (R // 2) * 8 + 2 * hd * 2
    sets = sets_for(nbytes)
    qn, kn = gen((hd,), 1.0, 0.1, dt, seed + 50), gen((hd,), 1.0, 0.1, dt, seed + 51)
    bufs = [(gen((1, T, hq, hd), 0.0, 1.0, dt, seed + 2 * k), gen((1, T, hk, hd), 0.0, 1.0, dt, seed + 2 * k + 1))
            for k in range(sets)]

    def launch(i):
        q, k = bufs[i % sets]
        ffi.rope_cs(q, q, k, k, table, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX)
    return Work(name, nbytes, launch, f"q/k head-norm + neox RoPE from a {{cos, sin}} table T={T} heads {hq}/{hk}",
                sets)


def make_qg_rope(name, fused, tokens=4096, hq=32, hk=4, hd=128, seed=640):
    """Qwen3.5 gated attention around the attention kernel: the q projection's interleaved [q | g] heads
    split (src/modules.rs:637-646), q / k head-norm (bias 1) + NeoX RoPE (669-681), and the output gate
    o *= sigmoid(g) (786).  Fused: exl3r_rope_qg reads q from qg and writes it dense, mul_sigmoid reads g
    in place from qg; unfused: deinterleave_qg, rope in place, mul_sigmoid on the dense g.  Both count the
    fused job's bytes: q read and written, k read and written, o and g read, o written, norm weights."""
    import numpy as np
    import torch
    import exl3r
    import exl3r.ffi as ffi
    f16 = torch.float16
    nbytes = 2 * tokens * hq * hd * 2 + 2 * tokens * hk * hd * 2 + 3 * tokens * hq * hd * 2 + 2 * hd * 2
    sets = sets_for(nbytes)
    inv = torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2, dtype=np.float64) / hd)).astype(np.float32)).cuda()
    qn, kn = gen((hd,), 0.0, 0.1, f16, seed + 50), gen((hd,), 0.0, 0.1, f16, seed + 51)
    n = tokens * hq
    bufs = [(gen((1, tokens, hq, 2 * hd), 0.0, 1.0, f16, seed + 3 * k), gen((1, tokens, hk, hd), 0.0, 1.0, f16, seed + 3 * k + 1),
             gen((n, hd), 0.0, 1.0, f16, seed + 3 * k + 2)) for k in range(sets)]
    q = torch.empty((1, tokens, hq, hd), device="cuda", dtype=f16)
    g = torch.empty((1, tokens, hq * hd), device="cuda", dtype=f16)

    def launch(i):
        qg, k, o = bufs[i % sets]
        if fused:
            ffi.rope_qg(qg, q, k, k, inv, 0, None, qn, kn, 1e-6, 1.0, exl3r.ROPE_NEOX, 1.0)
            ffi.mul_sigmoid(o, qg.view(n, 2 * hd)[:, hd:], o)
        else:
            ffi.deinterleave_qg(qg.view(1, tokens, hq * 2 * hd), q, g, hd)
            ffi.rope(q, q, k, k, inv, 0, None, qn, kn, 1e-6, 1.0, exl3r.ROPE_NEOX, 1.0)
            ffi.mul_sigmoid(o, g.view(n, hd), o)
    kind = "fused (rope_qg + gate read from qg)" if fused else "unfused (deinterleave + rope + gate)"
    return Work(name, nbytes, launch, f"gated attention q | g split + head-norm RoPE + output gate T={tokens} "
                                      f"heads {hq}/{hk} of {hd}, {kind}", sets)


def make_rope(name, pos, hq, hk, hd, R, mode, dt, seed, bsz=1, per_seq=False):
    import numpy as np
    import torch
    import exl3r
    import exl3r.ffi as ffi
    T = pos.size if not per_seq else bsz
    seq = T if not per_seq else 1
    b = 1 if not per_seq else bsz
    # q/k read + written, one int32 position per token, both norm weights, inv_freq.
    nbytes = 2 * T * (hq + hk) * hd * 2 + 4 * T + 2 * hd * 2 + (R // 2) * 4
    sets = sets_for(nbytes)
    inv = torch.from_numpy((1.0 / 1e6 ** (np.arange(0, R, 2, dtype=np.float64) / R)).astype(np.float32)).cuda()
    qn, kn = gen((hd,), 1.0, 0.1, dt, seed + 50), gen((hd,), 1.0, 0.1, dt, seed + 51)
    pos_d = torch.from_numpy(pos).cuda()
    bufs = [(gen((b, seq, hq, hd), 0.0, 1.0, dt, seed + 2 * k), gen((b, seq, hk, hd), 0.0, 1.0, dt, seed + 2 * k + 1))
            for k in range(sets)]
    m = exl3r.ROPE_NEOX if mode == "neox" else exl3r.ROPE_GPTJ

    def launch(i):
        q, k = bufs[i % sets]
        if per_seq:
            ffi.rope(q, q, k, k, inv, 0, pos_d, qn, kn, 1e-6, 0.0, m, 1.0)
        else:
            ffi.rope(q, q, k, k, inv, 0, None, qn, kn, 1e-6, 0.0, m, 1.0, position_ids=pos_d.view(1, -1))
    return Work(name, nbytes, launch, f"q/k head-norm + {mode} RoPE T={T} heads {hq}/{hk} hd {hd} rotary {R}", sets)


def make_gather(name, vocab, hidden, n, dt, out_dt, ids, seed, norm=False):
    import numpy as np
    import torch
    import exl3r.ffi as ffi
    table = gen((vocab, hidden), 0.0, 0.02, dt, seed)
    ids_d = torch.from_numpy(ids).cuda()
    es_o = torch.empty((), dtype=out_dt).element_size()
    distinct = len(np.unique(ids))
    if not norm:
        nbytes = n * hidden * (2 + es_o) + n * 8
        hbm = distinct * hidden * 2 + n * hidden * es_o + n * 8
        sets = sets_for(n * hidden * es_o)
        outs = [torch.empty((n, hidden), device="cuda", dtype=out_dt) for _ in range(sets)]

        def launch(i):
            ffi.embedding(table, ids_d, outs[i % sets])
        desc = f"embedding gather [{vocab},{hidden}] n={n}"
    else:
        w = gen((hidden,), 1.0, 0.1, dt, seed + 1)
        nbytes = n * hidden * 2 * 3 + n * 8 + hidden * 2
        hbm = distinct * hidden * 2 + n * hidden * 2 * 2 + n * 8 + hidden * 2
        sets = sets_for(2 * n * hidden * 2)
        outs = [(torch.empty((n, hidden), device="cuda", dtype=dt), torch.empty((n, hidden), device="cuda", dtype=dt))
                for _ in range(sets)]

        def launch(i):
            h, y = outs[i % sets]
            ffi.embedding_rms_norm(table, ids_d, h, w, y, 1e-6)
        desc = f"embedding gather + RMSNorm [{vocab},{hidden}] n={n} (h and y written)"
    return Work(name, nbytes, launch, f"{desc}, {distinct} distinct ids", sets, hbm_bytes=hbm)


def make_rope_kv(name, bsz, seq, fused, seed=400, max_blocks=64, had=False, cs=False, exact=False):
    """q/k head-norm + NeoX RoPE followed by the paged KV-cache append (64 q / 8 kv heads of 128, f16,
    256-token pages, positions = cache lengths): one fused exl3r_rope_paged_kv launch, or exl3r_rope
    then a separate append kernel (the reference's two launches).  With had, q / k / v are the raw
    projection outputs and their output rotations had_r_128(y, y, None, svh) (src/modules.rs:231) come
    first: one exl3r_rope_paged_kv_had launch (transforms on the matrix cores, or with exact the
    reference's butterfly), or three in-place rotations and the two launches.  With cs,
    the fused launch reads the forward pass's {cos, sin} table (exl3r_rope_cs_table, built once outside
    the timed launches) in place of evaluating sin / cos; its bytes count the table rows."""
    import numpy as np
    import torch
    import exl3r
    import exl3r.ffi as ffi
    hq, hk, hd, page = 64, 8, 128, 256
    T = bsz * seq
    # fused-op bytes: q, k read + written in place, v read, both cache rows written, positions
    nbytes = 2 * T * hq * hd * 2 + 2 * T * hk * hd * 2 + T * hk * hd * 2 + 2 * T * hk * hd * 2 + 4 * bsz + 2 * hd * 2
    if had:
        nbytes += (hq + 2 * hk) * hd * 2
    if cs:
        nbytes += T * (hd // 2) * 8 - 4 * bsz
    sets = sets_for(nbytes)
    rng = np.random.default_rng(seed)
    pages = bsz * max_blocks + 4
    bt = torch.from_numpy(rng.permutation(pages)[: bsz * max_blocks].reshape(bsz, max_blocks).astype(np.int32)).cuda()
    sl = torch.from_numpy(rng.integers(0, max_blocks * page - seq, bsz).astype(np.int32)).cuda()
    kc = torch.empty((pages, page, hk, hd), device="cuda", dtype=torch.float16)
    vc = torch.empty_like(kc)
    inv = torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2, dtype=np.float64) / hd)).astype(np.float32)).cuda()
    qn, kn = gen((hd,), 1.0, 0.1, torch.float16, seed + 1), gen((hd,), 1.0, 0.1, torch.float16, seed + 2)
    bufs = [tuple(gen((bsz, seq, h, hd), 0.0, 1.0, torch.float16, seed + 10 * j + i) for i, h in enumerate((hq, hk, hk)))
            for j in range(sets)]
    naive = exl3r.load_naive()
    sv = [torch.where(torch.rand(h * hd, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16) for h in (hq, hk, hk)]
    table = ffi.rope_cs_table(bsz, seq, inv, 0, sl) if cs else None

    def launch(i):
        q, k, v = bufs[i % sets]
        if had and fused:
            ffi.rope_paged_kv_had(q, q, k, k, v, inv, 0, sl, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, kc, vc, bt, sl,
                                  q_post_scale=sv[0], k_post_scale=sv[1], v_post_scale=sv[2], cs_table=table,
                                  exact=exact)
            return
        if had:
            for t, p in zip((q, k, v), sv):
                ffi.had_r_128(t.view(T, -1), t.view(T, -1), None, p)
        if fused:
            ffi.rope_paged_kv(q, q, k, k, v, inv, 0, sl, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, kc, vc, bt, sl,
                              cs_table=table)
        else:
            ffi.rope(q, q, k, k, inv, 0, sl, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
            rc = naive.naive_paged_kv_update_f16(k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
                                                 sl.data_ptr(), bsz, seq, hk, hd, max_blocks, page,
                                                 torch.cuda.current_stream().cuda_stream)
            assert rc == 0
    kind = "fused (1 launch)" if fused else "rope + separate append (2 launches)"
    if had:
        kind = "fused (1 launch)" if fused else "3 in-place rotations + rope + separate append (5 launches)"
    head = "q/k/v output rotation + " if had else ""
    if cs:
        kind += ", {cos, sin} table"
    return Work(name, nbytes, launch, f"{head}q/k norm + RoPE + paged KV append bsz {bsz} x {seq} tokens, {kind}", sets)


def make_gated(name, kind, tokens=4096, heads=32, hd=128, seed=600):
    """Qwen3.5-style gated ops over a prefill of `tokens`: the gated-delta-net output norm (bf16 core,
    f32 gate, f32 weight, f16 out, rows = tokens x heads of hd), the attention output gate
    x *= sigmoid(g) in place (f16 [tokens, heads * hd]), and the q | g split of the q projection."""
    import torch
    import exl3r.ffi as ffi
    n = tokens * heads * hd
    if kind == "norm":
        nbytes = n * (2 + 4 + 2) + hd * 4
        sets = sets_for(nbytes)
        bufs = [(gen((tokens * heads, hd), 0.0, 1.0, torch.bfloat16, seed + 3 * k),
                 gen((tokens * heads, hd), 0.0, 2.0, torch.float32, seed + 3 * k + 1),
                 torch.empty((tokens * heads, hd), device="cuda", dtype=torch.float16)) for k in range(sets)]
        w = gen((hd,), 1.0, 0.1, torch.float32, seed + 99)

        def launch(i):
            x, g, y = bufs[i % sets]
            ffi.gated_rms_norm(x, w, y, g, 1e-6, 0.0, 1, False, 0)
        desc = f"gated RMSNorm (silu gate) [{tokens * heads},{hd}] bf16 x, f32 g, f16 y"
    elif kind in ("norm_had", "norm_had_exact", "norm_had_unfused"):
        # ... feeding o_proj's input rotation (src/qwen3_5.rs:208-214): one fused launch (the transform on
        # the matrix cores, or the reference's butterfly), or the gated norm into y and exl3r_had_r_128;
        # all count the fused job's bytes
        nbytes = n * (2 + 4 + 2) + hd * 4 + heads * hd * 2
        sets = sets_for(nbytes)
        bufs = [(gen((tokens * heads, hd), 0.0, 1.0, torch.bfloat16, seed + 3 * k),
                 gen((tokens * heads, hd), 0.0, 2.0, torch.float32, seed + 3 * k + 1),
                 torch.empty((tokens, heads * hd), device="cuda", dtype=torch.float16)) for k in range(sets)]
        w = gen((hd,), 1.0, 0.1, torch.float32, seed + 99)
        suh = torch.where(torch.rand(heads * hd, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16)
        y = torch.empty((tokens * heads, hd), device="cuda", dtype=torch.float16)

        def launch(i):
            x, g, out = bufs[i % sets]
            if kind != "norm_had_unfused":
                ffi.gated_rms_norm_had(x, w, g, out.view(tokens * heads, hd), 1e-6, suh, pre_rows=heads,
                                       exact=kind == "norm_had_exact")
            else:
                ffi.gated_rms_norm(x, w, y, g, 1e-6, 0.0, 1, False, 0)
                ffi.had_r_128(y.view(tokens, heads * hd), out, suh)
        desc = (f"gated RMSNorm [{tokens * heads},{hd}] -> o_proj input rotation [{tokens},{heads * hd}], "
                f"{'unfused (gated norm + had_r_128)' if kind == 'norm_had_unfused' else 'fused'}"
                f"{', butterfly' if kind == 'norm_had_exact' else ''}")
    elif kind == "sigmoid":
        nbytes = 3 * n * 2
        sets = sets_for(nbytes)
        bufs = [(gen((tokens, heads * hd), 0.0, 1.0, torch.float16, seed + 2 * k),
                 gen((tokens, heads * hd), 0.0, 2.0, torch.float16, seed + 2 * k + 1)) for k in range(sets)]

        def launch(i):
            x, g = bufs[i % sets]
            ffi.mul_sigmoid_(x, g)
        desc = f"x *= sigmoid(g) in place [{tokens},{heads * hd}] f16"
    else:
        nbytes = 4 * n * 2
        sets = sets_for(nbytes)
        bufs = [(gen((tokens, heads * 2 * hd), 0.0, 1.0, torch.float16, seed + k),
                 torch.empty((tokens, heads, hd), device="cuda", dtype=torch.float16),
                 torch.empty((tokens, heads * hd), device="cuda", dtype=torch.float16)) for k in range(sets)]

        def launch(i):
            qg, q, g = bufs[i % sets]
            ffi.deinterleave_qg(qg, q, g, hd)
        desc = f"q | g deinterleave [{tokens},{heads},2x{hd}] f16"
    return Work(name, nbytes, launch, desc, sets)


def make_argmax(name, rows, use_torch, vocab=151936, seed=700, ws=False):
    """Greedy token choice over f16 logits [rows, vocab]: exl3r_argmax_sample (ws: its one-launch form
    exl3r_argmax_sample_ws), or torch.argmax on the same tensor (the generator's batched tch argmax, the
    reference's call path)."""
    import torch
    import exl3r.ffi as ffi
    nbytes = rows * vocab * 2 + rows * 8
    sets = sets_for(nbytes)
    bufs = [gen((rows, vocab), 0.0, 3.0, torch.float16, seed + k) for k in range(sets)]
    ids = torch.empty(rows, dtype=torch.int64, device="cuda")
    wsb = torch.zeros(ffi.sample_workspace_bytes(), dtype=torch.uint8, device="cuda") if ws else None

    def launch(i):
        x = bufs[i % sets]
        if use_torch:
            torch.argmax(x, dim=1, out=ids)
        elif ws:
            ffi.argmax_sample_ws(x, ids, wsb)
        else:
            ffi.argmax_sample(x, ids)
    what = "torch.argmax" if use_torch else "exl3r, one launch with a workspace" if ws else "exl3r"
    return Work(name, nbytes, launch, f"argmax over f16 logits [{rows},{vocab}] ({what})", sets)


def make_gumbel(name, rows, use_torch, vocab=151936, seed=720, ws=False):
    """Categorical draw from softmax(f16 logits [rows, vocab]): exl3r_gumbel_sample (Gumbel-max, one
    launch chain), or the reference sampler's tch path (src/sampler.rs:114: softmax, then
    multinomial(1, replacement)) on the same tensor."""
    import torch
    import exl3r.ffi as ffi
    nbytes = rows * vocab * 2 + rows * 8
    sets = sets_for(nbytes)
    bufs = [gen((rows, vocab), 0.0, 3.0, torch.float16, seed + k) for k in range(sets)]
    ids = torch.empty(rows, dtype=torch.int64, device="cuda")
    wsb = torch.zeros(ffi.sample_workspace_bytes(), dtype=torch.uint8, device="cuda") if ws else None

    def launch(i):
        x = bufs[i % sets]
        if use_torch:
            torch.multinomial(torch.softmax(x.float(), dim=-1), 1, True)
        elif ws:
            ffi.gumbel_sample_ws(x, ids, wsb, 0, i)
        else:
            ffi.gumbel_sample(x, ids, 0, i)
    what = "torch softmax + multinomial" if use_torch else \
        "exl3r Gumbel-max, one launch with a workspace" if ws else "exl3r Gumbel-max"
    return Work(name, nbytes, launch, f"categorical draw over f16 logits [{rows},{vocab}] ({what})", sets)


def make_had(name, rows, cols, seed=740, mfma=False):
    """EXL3 prefill input rotation: had_r_128 of f16 [rows, cols] with an f16 suh pre-scale (the
    projection input transform, src/modules.rs:227), out of place: the reference's butterfly
    (exl3r_had_r_128), or with mfma the matrix-core form (exl3r_had_r_128_mfma)."""
    import torch
    import exl3r.ffi as ffi
    nbytes = 2 * rows * cols * 2 + cols * 2
    sets = sets_for(nbytes)
    xs = [gen((rows, cols), 0.0, 1.0, torch.float16, seed + k) for k in range(sets)]
    outs = [torch.empty((rows, cols), device="cuda", dtype=torch.float16) for _ in range(sets)]
    suh = torch.where(torch.rand(cols, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16)

    def launch(i):
        ffi.had_r_128(xs[i % sets], outs[i % sets], suh, mfma=mfma)
    return Work(name, nbytes, launch, f"random-Hadamard row transform f16 [{rows},{cols}] with suh"
                + (", matrix cores" if mfma else ""), sets)


def make_norm_had(name, rows, cols, fused, seed=760, rotate=False, exact=False):
    """Qwen3-32B prefill attention input: r += x (f16 sublayer output into the f32 residual), the f16
    RMSNorm, and the q / k / v projections' input rotations had_r_128(y, suh_i)
    (src/modules.rs:224-227, 372-411): one fused launch, or the residual norm and three had_r_128
    launches.  With rotate, x is the previous projection's raw output and its own output rotation
    had_r_128(x, x, None, svh) (src/modules.rs:231) comes first (unfused: in place, one more launch).
    Both count the fused job's bytes (x, r read and written, three outputs, w, suh, svh).  The fused
    launch runs its transforms on the matrix cores, or with exact as the reference's butterfly; the
    unfused calls are the reference's (exl3r_had_r_128)."""
    import torch
    import exl3r.ffi as ffi
    n = rows * cols
    nbytes = n * (2 + 4 + 4 + 3 * 2) + (5 if rotate else 4) * cols * 2
    sets = sets_for(nbytes)
    bufs = [(gen((rows, cols), 0.0, 1.0, torch.float16, seed + 2 * k),
             gen((rows, cols), 0.0, 4.0, torch.float32, seed + 2 * k + 1),
             [torch.empty((rows, cols), device="cuda", dtype=torch.float16) for _ in range(3)]) for k in range(sets)]
    w = gen((cols,), 1.0, 0.1, torch.float16, seed + 99)
    suh = [torch.where(torch.rand(cols, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16) for _ in range(3)]
    y = torch.empty((rows, cols), device="cuda", dtype=torch.float16)
    svh = torch.where(torch.rand(cols, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16) if rotate else None

    def launch(i):
        x, r, outs = bufs[i % sets]
        if fused:
            ffi.rms_norm_had(x, w, outs, suh, 1e-6, r=r, rotate_x=rotate, x_post_scale=svh, exact=exact)
        else:
            if rotate:
                ffi.had_r_128(x, x, None, svh)
            ffi.rms_norm_res_in(x, w, y, r, 1e-6)
            for o, p in zip(outs, suh):
                ffi.had_r_128(y, o, p)
    kind = ("fused, butterfly" if exact else "fused") if fused else \
        f"unfused ({'had_r_128 in place + ' if rotate else ''}residual RMSNorm + 3 had_r_128)"
    head = "had(svh) -> residual RMSNorm" if rotate else "residual RMSNorm"
    return Work(name, nbytes, launch, f"{head} -> 3 Hadamard inputs [{rows},{cols}] f16/f32r, {kind}", sets)


def make_act_had(name, rows, cols, fused, seed=780, rotate=False, exact=False):
    """MLP prefill tail: silu(gate) * up in f16 and the down projection's input rotation
    had_r_128(a, suh) (src/modules.rs:932-940, 224-227): one fused launch, or exl3r_silu_mul and
    exl3r_had_r_128.  With rotate, gate and up are the raw gate_proj / up_proj outputs and their own
    output rotations (src/modules.rs:231) come first (unfused: two in-place rotations).  Both count the
    fused job's bytes (gate, up, the rotated output, suh, and svh of gate and up).  The fused launch runs
    its transforms on the matrix cores, or with exact as the reference's butterfly."""
    import torch
    import exl3r.ffi as ffi
    nbytes = rows * cols * 6 + (3 if rotate else 1) * cols * 2
    sets = sets_for(nbytes)
    bufs = [(gen((rows, cols), 0.0, 1.0, torch.float16, seed + 2 * k), gen((rows, cols), 0.0, 1.0, torch.float16, seed + 2 * k + 1),
             torch.empty((rows, cols), device="cuda", dtype=torch.float16)) for k in range(sets)]
    suh, sg, su = (torch.where(torch.rand(cols, device="cuda") < 0.5, -1.0, 1.0).to(torch.float16) for _ in range(3))
    a = torch.empty((rows, cols), device="cuda", dtype=torch.float16)

    def launch(i):
        g, u, out = bufs[i % sets]
        if fused:
            if rotate:
                ffi.act_mul_had("silu", g, u, out, suh, rotate_x=True, rotate_y=True, x_post_scale=sg, y_post_scale=su,
                                exact=exact)
            else:
                ffi.act_mul_had("silu", g, u, out, suh, exact=exact)
        else:
            if rotate:
                ffi.had_r_128(g, g, None, sg)
                ffi.had_r_128(u, u, None, su)
            ffi.silu_mul(g, u, a)
            ffi.had_r_128(a, out, suh)
    kind = ("fused, butterfly" if exact else "fused") if fused else \
        ("unfused (2 in-place rotations + silu_mul + had_r_128)" if rotate else
                                  "unfused (silu_mul + had_r_128)")
    head = "rotated gate, up -> " if rotate else ""
    return Work(name, nbytes, launch, f"{head}SiLU(gate)*up -> Hadamard input [{rows},{cols}] f16, {kind}", sets)


def make_prefill_layer(name, fused, T=4096, seed=900, cs=False):
    """The row ops and Hadamard rotations of one Qwen3-32B prefill layer (hidden 5120, 64 / 8 heads of
    128, intermediate 25600, f16 activations, f32 residual, 256-token pages), GEMMs and attention
    excluded.  Unfused, in the reference's order (src/modules.rs:224-231, 372-411, 669-704, 932-940,
    1020-1035): down_proj's output rotation, the residual norm, q / k / v input rotations, their output
    rotations, RoPE, the paged append, o_proj's input and output rotations, the residual norm, gate /
    up input rotations, their output rotations, silu_mul and down_proj's input rotation -- 20 launches.
    Fused: exl3r_rms_norm_had (rotate_x, 3 outputs), exl3r_rope_paged_kv_had, had_r_128 (o_proj input,
    after attention), exl3r_rms_norm_had (rotate_x, 2 outputs), exl3r_act_mul_had (both inputs
    rotated) -- 5 launches.  Bytes are the fused launches' algorithmic bytes."""
    import numpy as np
    import torch
    import exl3r
    import exl3r.ffi as ffi
    H, hq, hk, hd, I, page = 5120, 64, 8, 128, 25600, 256
    f16 = torch.float16

    def sgn(n):
        return torch.where(torch.rand(n, device="cuda") < 0.5, -1.0, 1.0).to(f16)
    r = gen((T, H), 0.0, 4.0, torch.float32, seed)
    y_down, y_o = gen((T, H), 0.0, 1.0, f16, seed + 1), gen((T, H), 0.0, 1.0, f16, seed + 2)
    q = gen((1, T, hq, hd), 0.0, 1.0, f16, seed + 3)
    k, v = gen((1, T, hk, hd), 0.0, 1.0, f16, seed + 4), gen((1, T, hk, hd), 0.0, 1.0, f16, seed + 5)
    o = gen((T, hq * hd), 0.0, 1.0, f16, seed + 6)
    g, u = gen((T, I), 0.0, 1.0, f16, seed + 7), gen((T, I), 0.0, 1.0, f16, seed + 8)
    w1, w2 = gen((H,), 1.0, 0.1, f16, seed + 9), gen((H,), 1.0, 0.1, f16, seed + 10)
    qn, kn = gen((hd,), 1.0, 0.1, f16, seed + 11), gen((hd,), 1.0, 0.1, f16, seed + 12)
    suh_q, suh_k, suh_v, suh_g, suh_u = sgn(H), sgn(H), sgn(H), sgn(H), sgn(H)
    svh_q, svh_k, svh_v, svh_o, svh_g, svh_u, svh_d = (sgn(hq * hd), sgn(hk * hd), sgn(hk * hd), sgn(H), sgn(I),
                                                       sgn(I), sgn(H))
    suh_o, suh_d = sgn(hq * hd), sgn(I)
    xq, xk, xv, xg, xu = (torch.empty((T, H), device="cuda", dtype=f16) for _ in range(5))
    xo = torch.empty((T, hq * hd), device="cuda", dtype=f16)
    xd, a = torch.empty((T, I), device="cuda", dtype=f16), torch.empty((T, I), device="cuda", dtype=f16)
    y = torch.empty((T, H), device="cuda", dtype=f16)
    max_blocks = T // page + 2
    pages = max_blocks + 2
    rng = np.random.default_rng(seed)
    bt = torch.from_numpy(rng.permutation(pages)[:max_blocks].reshape(1, max_blocks).astype(np.int32)).cuda()
    sl = torch.zeros(1, dtype=torch.int32, device="cuda")
    kc = torch.empty((pages, page, hk, hd), device="cuda", dtype=f16)
    vc = torch.empty_like(kc)
    inv = torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2, dtype=np.float64) / hd)).astype(np.float32)).cuda()
    naive = exl3r.load_naive()
    N = T * H
    nbytes = (N * (2 + 4 + 4 + 3 * 2) + 5 * H * 2                                     # norm -> q / k / v inputs
              + 2 * T * (hq + hk) * hd * 2 + T * hk * hd * 2 * 3 + 4 + 2 * hd * 2 + (hq + 2 * hk) * hd * 2   # rope + append
              + 2 * T * hq * hd * 2 + hq * hd * 2                                   # o_proj input rotation
              + N * (2 + 4 + 4 + 2 * 2) + 4 * H * 2                                 # norm -> gate / up inputs
              + T * I * 6 + 3 * I * 2)                                              # MLP tail

    table = ffi.rope_cs_table(1, T, inv, 0, sl) if cs else None

    def launch(i):
        if fused:
            ffi.rms_norm_had(y_down, w1, [xq, xk, xv], [suh_q, suh_k, suh_v], 1e-6, r=r, rotate_x=True,
                             x_post_scale=svh_d)
            ffi.rope_paged_kv_had(q, q, k, k, v, inv, 0, sl, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, kc, vc, bt, sl,
                                  q_post_scale=svh_q, k_post_scale=svh_k, v_post_scale=svh_v, cs_table=table)
            ffi.had_r_128(o, xo, suh_o)
            ffi.rms_norm_had(y_o, w2, [xg, xu], [suh_g, suh_u], 1e-6, r=r, rotate_x=True, x_post_scale=svh_o)
            ffi.act_mul_had("silu", g, u, xd, suh_d, rotate_x=True, rotate_y=True, x_post_scale=svh_g,
                            y_post_scale=svh_u)
            return
        ffi.had_r_128(y_down, y_down, None, svh_d)
        ffi.rms_norm_res_in(y_down, w1, y, r, 1e-6)
        for x_, s_ in ((xq, suh_q), (xk, suh_k), (xv, suh_v)):
            ffi.had_r_128(y, x_, s_)
        for t_, s_ in ((q, svh_q), (k, svh_k), (v, svh_v)):
            ffi.had_r_128(t_.view(T, -1), t_.view(T, -1), None, s_)
        ffi.rope(q, q, k, k, inv, 0, sl, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
        rc = naive.naive_paged_kv_update_f16(k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
                                             sl.data_ptr(), 1, T, hk, hd, max_blocks, page,
                                             torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        ffi.had_r_128(o, xo, suh_o)
        ffi.had_r_128(y_o, y_o, None, svh_o)
        ffi.rms_norm_res_in(y_o, w2, y, r, 1e-6)
        for x_, s_ in ((xg, suh_g), (xu, suh_u)):
            ffi.had_r_128(y, x_, s_)
        ffi.had_r_128(g, g, None, svh_g)
        ffi.had_r_128(u, u, None, svh_u)
        ffi.silu_mul(g, u, a)
        ffi.had_r_128(a, xd, suh_d)
    kind = "fused (5 launches)" if fused else "unfused, the reference's order (20 launches)"
    return Work(name, nbytes, launch, f"Qwen3-32B prefill layer row ops + rotations T={T}, {kind}")


def make_copy(name, cached=False):
    import torch
    import exl3r
    nb = 1 << 30
    src = torch.empty(nb, dtype=torch.uint8, device="cuda")
    dst = torch.empty(nb, dtype=torch.uint8, device="cuda")
    naive = exl3r.load_naive()
    fn = naive.calib_copy_cached if cached else naive.calib_copy

    def launch(i):
        rc = fn(src.data_ptr(), dst.data_ptr(), nb, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
    return Work(name, 2 * nb, launch, f"{'cached' if cached else 'non-temporal'} copy 1 GiB (counter calibration)")


def make_decode(fused, seed=7):
    """One layer of a 64-row decode step, fp16: attn-norm (residual) + q/k head-norm + RoPE +
    mlp-norm (residual) + SiLU-mul, fused (4 launches) or naive unfused (10 launches)."""
    import numpy as np
    import torch
    import exl3r
    T, H, I, hq, hk, hd = 64, 5120, 17408, 64, 8, 128
    f16 = torch.float16
    resid = gen((T, H), 0.0, 4.0, f16, seed)
    a_out = gen((T, H), 0.0, 1.0, f16, seed + 1)
    m_out = gen((T, H), 0.0, 1.0, f16, seed + 2)
    w1, w2 = gen((H,), 1.0, 0.1, f16, seed + 3), gen((H,), 1.0, 0.1, f16, seed + 4)
    y = torch.empty((T, H), device="cuda", dtype=f16)
    q = gen((T, 1, hq, hd), 0.0, 1.0, f16, seed + 5)
    k = gen((T, 1, hk, hd), 0.0, 1.0, f16, seed + 6)
    qn, kn = gen((hd,), 1.0, 0.1, f16, seed + 7), gen((hd,), 1.0, 0.1, f16, seed + 8)
    pos = torch.from_numpy(np.random.default_rng(seed).integers(0, 32768, T).astype(np.int32)).cuda()
    inv = torch.from_numpy((1.0 / 1e6 ** (np.arange(0, hd, 2, dtype=np.float64) / hd)).astype(np.float32)).cuda()
    gate, up = gen((T, I), 0.0, 1.0, f16, seed + 9), gen((T, I), 0.0, 1.0, f16, seed + 10)
    act = torch.empty((T, I), device="cuda", dtype=f16)
    nbytes = 2 * (4 * T * H * 2 + H * 2) + (2 * T * (hq + hk) * hd * 2 + 4 * T + 2 * hd * 2 + hd * 2) + 3 * T * I * 2
    P = lambda t: t.data_ptr()
    if fused:
        # Both variants call their C ABI directly with pre-bound arguments (as a compiled caller
        # would), so the eager timing compares launches, not Python wrapper overhead.
        lib = exl3r.load()
        F16 = exl3r.F16

        def launch(i):
            s = torch.cuda.current_stream().cuda_stream
            rc = lib.exl3r_rms_norm_res_in(P(a_out), F16, H, P(w1), F16, P(y), F16, H, P(resid), F16, H,
                                           T, H, 1e-6, 0.0, 1.0, s)
            rc |= lib.exl3r_rope(P(q), P(q), hq * hd, hd, hq, P(k), P(k), hk * hd, hd, hk, F16, T, 1, hd,
                                 P(inv), hd, 0, P(pos), None, P(qn), P(kn), F16, 1e-6, 0.0,
                                 exl3r.ROPE_NEOX, 1.0, s)
            rc |= lib.exl3r_rms_norm_res_in(P(m_out), F16, H, P(w2), F16, P(y), F16, H, P(resid), F16, H,
                                            T, H, 1e-6, 0.0, 1.0, s)
            rc |= lib.exl3r_silu_mul(P(gate), P(up), F16, P(act), F16, T, I, I, I, I, 0.0, s)
            assert rc == 0
        return Work("decode_fused", nbytes, launch, "decode layer T=64 fused (4 launches)")
    naive = exl3r.load_naive()
    tmp = torch.empty((T, I), device="cuda", dtype=f16)

    def launch(i):
        s = torch.cuda.current_stream().cuda_stream
        rc = naive.naive_add_f16(P(a_out), P(resid), P(resid), T * H, s)
        rc |= naive.naive_rms_norm_f16(P(resid), P(w1), P(y), T, H, 1e-6, s)
        rc |= naive.naive_head_norm_f16(P(q), P(qn), T, hq, hd, 1e-6, s)
        rc |= naive.naive_head_norm_f16(P(k), P(kn), T, hk, hd, 1e-6, s)
        rc |= naive.naive_rope_neox_f16(P(q), P(inv), P(pos), T, 1, hq, hd, s)
        rc |= naive.naive_rope_neox_f16(P(k), P(inv), P(pos), T, 1, hk, hd, s)
        rc |= naive.naive_add_f16(P(m_out), P(resid), P(resid), T * H, s)
        rc |= naive.naive_rms_norm_f16(P(resid), P(w2), P(y), T, H, 1e-6, s)
        rc |= naive.naive_silu_f16(P(gate), P(tmp), T * I, s)
        rc |= naive.naive_mul_f16(P(tmp), P(up), P(act), T * I, s)
        assert rc == 0
    return Work("decode_naive", nbytes, launch, "decode layer T=64 naive unfused (10 launches)")


def make_all(only=None):
    import torch
    bf16, f16 = torch.bfloat16, torch.float16
    ragged = ragged_positions(0)
    builders = {
        "rms_c3": lambda: make_rms("rms_c3", 8192, 5120, bf16, True, 100),
        "rms_q3mix": lambda: make_rms("rms_q3mix", 8192, 5120, f16, True, 110, rdt=torch.float32),
        "silu_c3": lambda: make_act("silu_c3", 8192, 17408, bf16, "silu", 200),
        "gelu_c3": lambda: make_act("gelu_c3", 8192, 17408, bf16, "gelu", 200),
        "rope_c4": lambda: make_rope("rope_c4", ragged, 64, 8, 128, 128, "neox", f16, 300),
        "rope_c4_gptj": lambda: make_rope("rope_c4_gptj", ragged, 64, 8, 128, 64, "gptj", f16, 310),
        "rope_cs_c4": lambda: make_rope_cs("rope_cs_c4", ragged, 64, 8, 128, 128, f16, 300, False),
        "rope_cs_table_c4": lambda: make_rope_cs("rope_cs_table_c4", ragged, 64, 8, 128, 128, f16, 300, True),
        "qg_rope_q35": lambda: make_qg_rope("qg_rope_q35", True),
        "rope_kv_prefill_cs": lambda: make_rope_kv("rope_kv_prefill_cs", 1, 4096, True, cs=True),
        "rope_kv_had_prefill_cs": lambda: make_rope_kv("rope_kv_had_prefill_cs", 1, 4096, True, had=True, cs=True),
        "prefill_layer_cs": lambda: make_prefill_layer("prefill_layer_cs", True, cs=True),
        "qg_rope_q35_unfused": lambda: make_qg_rope("qg_rope_q35_unfused", False),
        "gather_c5": lambda: make_gather("gather_c5", 151936, 5120, 16384, bf16, bf16, zipf_ids(16384, 151936, 1), 400),
        "gather_f32_c5": lambda: make_gather("gather_f32_c5", 151936, 5120, 16384, bf16, torch.float32,
                                             zipf_ids(16384, 151936, 1), 400),
        "gather_norm_c5": lambda: make_gather("gather_norm_c5", 151936, 5120, 16384, bf16, bf16,
                                              zipf_ids(16384, 151936, 1), 400, norm=True),
        "rms_c1": lambda: make_rms("rms_c1", 512, 1024, f16, False, 500),
        "silu_c1": lambda: make_act("silu_c1", 512, 3072, f16, "silu", 510),
        "rope_c1": lambda: make_rope("rope_c1", __import__("numpy").arange(512, dtype="int32"), 16, 8, 128, 128, "neox",
                                     f16, 520),
        "gather_c1": lambda: make_gather("gather_c1", 151936, 1024, 512, f16, f16,
                                         __import__("numpy").random.default_rng(0).integers(0, 151936, 512), 530),
        "decode_fused": lambda: make_decode(True),
        "decode_naive": lambda: make_decode(False),
        "rope_kv_prefill": lambda: make_rope_kv("rope_kv_prefill", 1, 4096, True),
        "rope_kv_prefill_unfused": lambda: make_rope_kv("rope_kv_prefill_unfused", 1, 4096, False),
        "rope_kv_dec": lambda: make_rope_kv("rope_kv_dec", 64, 1, True, max_blocks=16),
        "rope_kv_dec_unfused": lambda: make_rope_kv("rope_kv_dec_unfused", 64, 1, False, max_blocks=16),
        "gated_norm_q35": lambda: make_gated("gated_norm_q35", "norm"),
        "mul_sigmoid_q35": lambda: make_gated("mul_sigmoid_q35", "sigmoid"),
        "deinterleave_q35": lambda: make_gated("deinterleave_q35", "deinterleave"),
        "gated_norm_had_q35": lambda: make_gated("gated_norm_had_q35", "norm_had"),
        "gated_norm_had_q35_unfused": lambda: make_gated("gated_norm_had_q35_unfused", "norm_had_unfused"),
        "gated_norm_had_q35_exact": lambda: make_gated("gated_norm_had_q35_exact", "norm_had_exact"),
        "argmax_dec": lambda: make_argmax("argmax_dec", 64, False),
        "argmax_dec_torch": lambda: make_argmax("argmax_dec_torch", 64, True),
        "argmax_dec_ws": lambda: make_argmax("argmax_dec_ws", 64, False, ws=True),
        "argmax_prefill": lambda: make_argmax("argmax_prefill", 1024, False),
        "argmax_prefill_torch": lambda: make_argmax("argmax_prefill_torch", 1024, True),
        "gumbel_dec": lambda: make_gumbel("gumbel_dec", 64, False),
        "gumbel_dec_ws": lambda: make_gumbel("gumbel_dec_ws", 64, False, ws=True),
        "gumbel_dec_torch": lambda: make_gumbel("gumbel_dec_torch", 64, True),
        "gumbel_prefill": lambda: make_gumbel("gumbel_prefill", 1024, False),
        "had_c3": lambda: make_had("had_c3", 8192, 5120),
        "had_c3_mfma": lambda: make_had("had_c3_mfma", 8192, 5120, mfma=True),
        "norm_had_c3": lambda: make_norm_had("norm_had_c3", 8192, 5120, True),
        "norm_had_c3_exact": lambda: make_norm_had("norm_had_c3_exact", 8192, 5120, True, exact=True),
        "norm_had_c3_unfused": lambda: make_norm_had("norm_had_c3_unfused", 8192, 5120, False),
        "norm_had_rot_c3": lambda: make_norm_had("norm_had_rot_c3", 8192, 5120, True, rotate=True),
        "norm_had_rot_c3_exact": lambda: make_norm_had("norm_had_rot_c3_exact", 8192, 5120, True, rotate=True,
                                                       exact=True),
        "norm_had_rot_c3_unfused": lambda: make_norm_had("norm_had_rot_c3_unfused", 8192, 5120, False, rotate=True),
        "rope_kv_had_prefill": lambda: make_rope_kv("rope_kv_had_prefill", 1, 4096, True, had=True),
        "rope_kv_had_prefill_unfused": lambda: make_rope_kv("rope_kv_had_prefill_unfused", 1, 4096, False, had=True),
        "rope_kv_had_prefill_exact": lambda: make_rope_kv("rope_kv_had_prefill_exact", 1, 4096, True, had=True,
                                                          exact=True),
        "rope_had_c4": lambda: make_rope_had("rope_had_c4", ragged, 64, 8, 128, True),
        "rope_had_c4_exact": lambda: make_rope_had("rope_had_c4_exact", ragged, 64, 8, 128, True, exact=True),
        "rope_had_c4_unfused": lambda: make_rope_had("rope_had_c4_unfused", ragged, 64, 8, 128, False),
        "prefill_layer": lambda: make_prefill_layer("prefill_layer", True),
        "prefill_layer_unfused": lambda: make_prefill_layer("prefill_layer_unfused", False),
        "mlp_had_c3": lambda: make_act_had("mlp_had_c3", 8192, 17408, True, rotate=True),
        "mlp_had_c3_exact": lambda: make_act_had("mlp_had_c3_exact", 8192, 17408, True, rotate=True, exact=True),
        "mlp_had_c3_unfused": lambda: make_act_had("mlp_had_c3_unfused", 8192, 17408, False, rotate=True),
        "silu_had_c3": lambda: make_act_had("silu_had_c3", 8192, 17408, True),
        "silu_had_c3_exact": lambda: make_act_had("silu_had_c3_exact", 8192, 17408, True, exact=True),
        "silu_had_c3_unfused": lambda: make_act_had("silu_had_c3_unfused", 8192, 17408, False),
        "calib_copy": lambda: make_copy("calib_copy"),
        "calib_copy_cached": lambda: make_copy("calib_copy_cached", cached=True),
    }
    names = ([only] if isinstance(only, str) else list(only)) if only else \
        [n for n in OPS if n not in ("rms_c2", "calib_copy_cached", "c3_step")]
    return {n: builders[n]() for n in names}


# ------------------------------------------------------------------------------------------------
# Timing

def time_launches(work, steps, warmup):
    """Average duration of one launch (ms): HIP events on the launch stream around `steps`
    back-to-back launches."""
    import torch
    for i in range(warmup):
        work.launch(i)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(steps):
        work.launch(warmup + i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def time_graph(work, per_graph=20, replays=10):
    """Per-launch time with the launches captured in a HIP graph (no host launch overhead)."""
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(per_graph):
            work.launch(i)
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / (per_graph * replays)


def rms_c2_latencies():
    """Config 2: decode-batch residual RMSNorm, f16, hidden 5120, T in {1, 8, 32, 64}: us per call,
    eager (back-to-back launches) and inside a HIP graph."""
    import torch
    out = {}
    for T in (1, 8, 32, 64):
        w = make_rms(f"rms_c2_t{T}", T, 5120, torch.float16, True, 600 + T)
        eager = time_launches(w, 200, 20) * 1000
        graph = time_graph(w, 50, 10) * 1000
        out[str(T)] = {"us_eager": round(eager, 3), "us_graph": round(graph, 3), "bytes": w.nbytes,
                       "gbs_graph": round(w.nbytes / (graph * 1e-6) / 1e9, 1)}
    return out


# ------------------------------------------------------------------------------------------------
# CPU baseline (the oracle, timed on this host)

def cpu_threads():
    """Threads of the CPU baseline: every core of the process affinity mask, capped by OMP_NUM_THREADS
    when the environment sets it (the GPU boxes set it to the process's CPU share, 16 per GPU)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return (min(aff, int(omp)) if omp.isdigit() and int(omp) > 0 else aff), aff


def cpu_baseline(seconds):
    """The CPU oracle (C, OpenMP; the reference has no CPU path for these ops) timed on this host over
    every BASELINE config and the decode composite, each config on the sample named in its entry, with
    outputs preallocated (the oracle's C entry points are called directly).  Per config: one warm-up,
    then repetitions until its share of `seconds` is spent (at least 5); the median is reported.  The
    headline `value` is the C3 step sample (the bench's own workload)."""
    import ctypes
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    lib = orc.load()
    nthreads, aff = cpu_threads()
    rng = np.random.default_rng(0)
    P = orc._p
    F16, BF16, F32 = orc.F16, orc.BF16, orc.F32

    def normal(shape, mean, std, code):
        return orc.to_bits(rng.standard_normal(shape, dtype=np.float32) * std + mean, code)

    def empty(shape, code):
        return np.empty(shape, orc.storage_dtype(code))

    def res_norm(T, H, dt):
        x, r0, w = normal((T, H), 0, 1, dt), normal((T, H), 0, 4, dt), normal((H,), 1, 0.1, dt)
        r, y = r0.copy(), empty((T, H), dt)

        def run():   # r accumulates x over the reps (values stay finite: the timing does not depend on them)
            lib.oracle_rms_norm(P(x), dt, H, P(w), dt, P(y), dt, H, P(r), dt, H, T, H, 1e-6, 0.0, 1.0, nthreads)
        return run, 4 * T * H * 2 + H * 2

    def norm(T, H, dt):
        x, w, y = normal((T, H), 0, 1, dt), normal((H,), 1, 0.1, dt), empty((T, H), dt)

        def run():
            lib.oracle_rms_norm(P(x), dt, H, P(w), dt, P(y), dt, H, None, F32, H, T, H, 1e-6, 0.0, 1.0, nthreads)
        return run, 2 * T * H * 2 + H * 2

    def act(T, I, dt, a):
        g, u, z = normal((T, I), 0, 1, dt), normal((T, I), 0, 1, dt), empty((T, I), dt)

        def run():
            lib.oracle_act_mul(a, P(g), P(u), dt, P(z), dt, T, I, I, I, I, 0.0, nthreads)
        return run, 3 * T * I * 2

    def rope(pos, hq, hk, hd, R, mode):
        T = pos.size
        q, k = normal((1, T, hq, hd), 0, 1, F16), normal((1, T, hk, hd), 0, 1, F16)
        qn, kn = normal((hd,), 1, 0.1, F16), normal((hd,), 1, 0.1, F16)
        oq, ok = empty(q.shape, F16), empty(k.shape, F16)
        inv = (1.0 / 1e6 ** (np.arange(0, R, 2, dtype=np.float64) / R)).astype(np.float32)
        pid = np.ascontiguousarray(pos.reshape(1, T), np.int32)

        def run():
            lib.oracle_rope(P(q), P(oq), hq * hd, hd, hq, P(k), P(ok), hk * hd, hd, hk, F16, 1, T, hd, P(inv), R, 0,
                            None, P(pid), P(qn), P(kn), F16, 1e-6, 0.0, mode, 1.0, nthreads)
        return run, 2 * T * (hq + hk) * hd * 2 + 4 * T + 2 * hd * 2 + (R // 2) * 4

    def gather(vocab, H, ids, dt, with_norm):
        table = np.zeros((vocab, H), orc.storage_dtype(dt))    # values do not change the work; rows touched once
        table[np.unique(ids)] = normal((np.unique(ids).size, H), 0, 0.02, dt)
        ids = np.ascontiguousarray(ids, np.int64)
        n = ids.size
        w, h, y = normal((H,), 1, 0.1, dt), empty((n, H), dt), empty((n, H), dt)
        err = np.zeros(1, np.int32)
        if with_norm:
            def run():
                lib.oracle_embedding_rms_norm(P(table), dt, vocab, H, H, P(ids), orc.I64, n, P(h), dt, H, P(w), dt,
                                              P(y), dt, H, 1e-6, 0.0, 1.0, P(err), nthreads)
            return run, n * H * 2 * 3 + n * 8 + H * 2
        def run():
            lib.oracle_embedding(P(table), dt, vocab, H, H, P(ids), orc.I64, n, P(h), dt, H, P(err), nthreads)
        return run, n * H * 2 * 2 + n * 8

    ragged = ragged_positions(0)
    cases = {
        "c1_rms_norm": ("full C1: RMSNorm [512,1024] f16", lambda: norm(512, 1024, F16)),
        "c1_silu_mul": ("full C1: SiLU-mul [512,3072] f16", lambda: act(512, 3072, F16, orc.ACT_SILU)),
        "c1_rope": ("full C1: q/k head-norm + NeoX RoPE, 512 tokens, 16/8 heads of 128, f16",
                    lambda: rope(np.arange(512, dtype=np.int32), 16, 8, 128, 128, orc.ROPE_NEOX)),
        "c1_gather": ("full C1: gather of 512 uniform ids from [151936,1024] f16",
                      lambda: gather(151936, 1024, np.random.default_rng(0).integers(0, 151936, 512), F16, False)),
        "c2_res_norm_t64": ("full C2 at T=64: residual RMSNorm [64,5120] f16", lambda: res_norm(64, 5120, F16)),
        "c3_res_norm": ("C3 row sample: residual RMSNorm [256,5120] bf16", lambda: res_norm(256, 5120, BF16)),
        "c3_silu_mul": ("C3 row sample: SiLU-mul [64,17408] bf16", lambda: act(64, 17408, BF16, orc.ACT_SILU)),
        "c3_gelu_mul": ("C3 row sample: GELU-mul [64,17408] bf16", lambda: act(64, 17408, BF16, orc.ACT_GELU)),
        "c4_rope_neox": ("C4 token sample: the first 512 of the ragged tokens, 64/8 heads of 128, NeoX, f16",
                         lambda: rope(ragged[:512], 64, 8, 128, 128, orc.ROPE_NEOX)),
        "c4_rope_gptj": ("C4 token sample: 512 tokens, GPT-J at rotary_dim 64",
                         lambda: rope(ragged[:512], 64, 8, 128, 64, orc.ROPE_GPTJ)),
        "c5_gather_norm": ("C5 id sample: gather + RMSNorm of 1024 Zipf ids from [151936,5120] bf16 (h and y)",
                           lambda: gather(151936, 5120, zipf_ids(1024, 151936, 1), BF16, True)),
    }
    out = {}
    share = seconds / (len(cases) + 1)
    for name, (sample, build) in cases.items():
        run, nbytes = build()
        run()
        times = []
        t_end = time.perf_counter() + share
        while time.perf_counter() < t_end or len(times) < 5:
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        out[name] = {"us": round(med * 1e6, 2), "gbs": round(nbytes / med / 1e9, 3), "bytes": nbytes,
                     "reps": len(times), "sample": sample}
    # the 64-row decode layer: the sum of its four ops (2 residual norms, RoPE, SiLU-mul), f16
    runs = [res_norm(64, 5120, F16), res_norm(64, 5120, F16),
            rope(np.random.default_rng(7).integers(0, 32768, 64).astype(np.int32), 64, 8, 128, 128, orc.ROPE_NEOX),
            act(64, 17408, F16, orc.ACT_SILU)]
    for r, _ in runs:
        r()
    times = []
    t_end = time.perf_counter() + share
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        for r, _ in runs:
            r()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    nb = sum(b for _, b in runs)
    out["decode_layer_t64"] = {"us": round(med * 1e6, 2), "gbs": round(nb / med / 1e9, 3), "bytes": nb,
                               "reps": len(times), "sample": "full: 64-row decode layer, 2 residual norms + RoPE + SiLU-mul, f16"}
    c3 = [out[k] for k in ("c3_res_norm", "c3_silu_mul", "c3_gelu_mul")]
    c3_gbs = sum(c["bytes"] for c in c3) / (sum(c["us"] for c in c3) * 1e-6) / 1e9
    return {"value": round(c3_gbs, 3), "unit": "GB/s", "cores": nthreads, "affinity_cores": aff, "kind": "port",
            "sample": (f"value: the C3 step on a row sample (residual RMSNorm [256,5120] + SiLU-mul and GELU-mul "
                       f"[64,17408] bf16); the CPU oracle (C, OpenMP, {nthreads} threads of {aff} in the affinity "
                       f"mask), median per config over ~{share:.1f} s each; every config in `configs`"),
            "configs": out}


def decode_eager_compiled(timeout=120):
    """Runs the compiled eager decode-layer timing (exllamav3-rs_amd/bin/exl3r_bench_decode) as a child
    process and returns its JSON, or None (with the reason logged) when it is not built or fails."""
    import subprocess
    exe = os.path.join(ROOT, "exllamav3-rs_amd", "bin", "exl3r_bench_decode")
    if not os.path.exists(exe):
        log(f"decode eager (compiled): {exe} is not built")
        return None
    try:
        p = subprocess.run([exe, "2000", "7"], capture_output=True, text=True, timeout=timeout)
    except subprocess.TimeoutExpired:
        log("decode eager (compiled): timed out")
        return None
    if p.returncode != 0:
        log(f"decode eager (compiled): exit {p.returncode}: {p.stderr.strip()[-300:]}")
        return None
    res = json.loads(p.stdout.strip().splitlines()[-1])
    res["timing"] = ("median of 7 windows of 2000 layers enqueued back to back from C++ (host layer ffi wrappers "
                     "with their argument checks / the naive C entry points), HIP events on the stream")
    log(f"decode eager (compiled): fused {res['fused_us']:.2f} us vs naive {res['naive_us']:.2f} us "
        f"(x{res['speedup']:.2f}); host enqueue {res['fused_host_enqueue_us']:.2f} / {res['naive_host_enqueue_us']:.2f} us")
    return res


def pmc_kib(op, counter, timeout=120):
    """Median KiB per dispatch of a rocprofv3 counter for each of this library's kernels in
    `bench.py --op OP` (a child process under rocprofv3 --pmc, one counter per run), or None when the
    profiler is missing or the run fails."""
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(exe):
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "run", "--", sys.executable,
               os.path.abspath(__file__), "--op", op, "--steps", "5", "--warmup", "1"]
        p = subprocess.Popen(cmd, cwd="/tmp", stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                             env={**os.environ, "TMPDIR": "/tmp"}, start_new_session=True)
        try:
            rc = p.wait(timeout=timeout)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.wait()
            return None
        files = glob.glob(os.path.join(d, "**", "run_counter_collection.csv"), recursive=True)
        if rc != 0 and not files:
            return None
        vals = {}
        for f in files:
            for r in csv.DictReader(open(f)):
                k = r.get("Kernel_Name", "")
                if "exl3r::" in k or "k_calib" in k:
                    vals.setdefault(k, []).append(float(r["Counter_Value"]))
        return {k: statistics.median(v) for k, v in vals.items()} or None


def trace_step(steps, warmup, timeout=150):
    """Each C3 step kernel's median duration (us) inside the step sequence: a rocprofv3 --kernel-trace run of
    `bench.py --op c3_step` (the three launches back to back, as in the timed step), the warmup launches
    dropped (the median: one dispatch delayed by the profiler does not move it).  None when the profiler
    is missing or the run fails."""
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(exe):
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        cmd = [exe, "--kernel-trace", "--output-format", "csv", "-d", d, "-o", "run", "--", sys.executable,
               os.path.abspath(__file__), "--op", "c3_step", "--steps", str(steps), "--warmup", str(warmup)]
        p = subprocess.Popen(cmd, cwd="/tmp", stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                             env={**os.environ, "TMPDIR": "/tmp"}, start_new_session=True)
        try:
            p.wait(timeout=timeout)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.wait()
            return None
        files = glob.glob(os.path.join(d, "**", "run_kernel_trace.csv"), recursive=True)
        durs = {n: [] for n in STEP_OPS}
        for f in files:
            rows = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Start_Timestamp"]))
            for r in rows:
                k = r.get("Kernel_Name", "")
                n = "rms_c3" if "k_rms_norm" in k else "silu_c3" if "k_act_mul<0," in k else \
                    "gelu_c3" if "k_act_mul<1," in k else None
                if n:
                    durs[n].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        out = {n: statistics.median(v[warmup:]) for n, v in durs.items() if len(v) > warmup}
        return out or None


def live_traffic(op):
    """HBM bytes per launch of op's main kernel counted in this run: FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch, one rocprofv3 --pmc run each), scaled by what the same counters read for a plain copy of
    1 GiB read + 1 GiB write (calib_copy).  Returns (bytes, kernel name, detail) or None."""
    cf, cw = pmc_kib("calib_copy", "FETCH_SIZE"), pmc_kib("calib_copy", "WRITE_SIZE")
    f, w = pmc_kib(op, "FETCH_SIZE"), pmc_kib(op, "WRITE_SIZE")
    if not (cf and cw and f and w):
        return None
    fs = (1 << 30) / (max(cf.values()) * 1024)
    ws = (1 << 30) / (max(cw.values()) * 1024)
    per = {k: f[k] * 1024 * fs + w.get(k, 0.0) * 1024 * ws for k in f}
    k = max(per, key=per.get)
    return int(per[k]), k, {"fetch_kib": round(f[k], 1), "write_kib": round(w.get(k, 0.0), 1),
                            "fetch_scale": round(fs, 4), "write_scale": round(ws, 4)}


def traffic_from_profiles(op):
    """HBM bytes per launch of the op's main kernel from the committed rocprofv3 --pmc summary, or None
    (an op with a second, small kernel -- the {cos, sin} table -- has a line for each: the larger is kept)."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.txt")
    if not os.path.exists(path):
        return None
    best = None
    for line in open(path):
        parts = line.split()
        if len(parts) >= 2 and parts[0] == op + ":":
            kv = dict(p.split("=", 1) for p in parts[1:] if "=" in p)
            if "traffic_bytes" in kv:
                t = int(float(kv["traffic_bytes"]))
                best = t if best is None else max(best, t)
    return best


# ------------------------------------------------------------------------------------------------

def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the row ops are "
              "token-independent and would shard over tokens with no exchange -- run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    # The eager decode layer timed from compiled code (a child process, started before this process
    # touches the GPU): the reference's batched decode is not graph-captured.
    dec_compiled = None if args.op else decode_eager_compiled()
    import torch
    import exl3r
    exl3r.load()
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        if args.op == "c3_step":
            # the timed step's launch sequence on its own (rocprofv3 kernel-trace runs)
            ws = make_all(STEP_OPS)
            for i in range(args.warmup + args.steps):
                for n in STEP_OPS:
                    ws[n].launch(i)
            torch.cuda.synchronize()
            log(f"c3_step: {args.warmup + args.steps} steps launched")
            return
        if args.op:
            work = make_all(args.op)[args.op] if args.op != "rms_c2" else None
            if work is None:
                log(json.dumps(rms_c2_latencies()))
                return
            ms = time_launches(work, args.steps, args.warmup)
            log(f"{work.name}: {work.desc}: {ms * 1000:.2f} us/launch, {work.nbytes / (ms * 1e-3) / 1e9:.1f} GB/s")
            return

        works = make_all()
        torch.cuda.synchronize()
        ops = {}
        for name, w in works.items():
            if name == "calib_copy":
                continue
            steps = max(args.steps, 50) if name.endswith("_c1") or name.startswith("decode") else args.steps
            # median of three timed windows of `steps` launches (the first window after a different
            # workload can run at a lower clock); the minimum is kept beside it
            windows = sorted(time_launches(w, steps, args.warmup if k == 0 else 0) for k in range(3))
            ms = windows[1]
            gbs = w.nbytes / (ms * 1e-3) / 1e9
            ops[name] = {"desc": w.desc, "us": round(ms * 1000, 3), "us_min": round(windows[0] * 1000, 3),
                         "bytes": w.nbytes, "gbs": round(gbs, 1), "frac_peak": round(gbs / PEAK_GBS, 4)}
            if w.hbm_bytes is not None:
                # repeats are cache hits: the HBM fraction is over the least traffic that serves the launch
                # (each distinct row read once, computed from this run's ids); the all-rows rate stays beside
                # it as gbs, and the committed rocprofv3 FETCH/WRITE count (a row read by workgroups on
                # several XCDs is fetched into each XCD's L2) beside that, with its source
                hbm_gbs = w.hbm_bytes / (ms * 1e-3) / 1e9
                ops[name].update({"hbm_bytes": w.hbm_bytes, "hbm_bytes_source": "distinct rows (lower bound)",
                                  "hbm_gbs": round(hbm_gbs, 1), "frac_peak": round(hbm_gbs / PEAK_GBS, 4)})
                counted = traffic_from_profiles(name)
                if counted:
                    ops[name].update({"hbm_bytes_profiled": counted,
                                      "hbm_bytes_profiled_source": "profiles/pmc_traffic.txt (committed counters)"})
                gbs = hbm_gbs
            extra = ""
            if name.endswith("_c1") or name.startswith("rope_kv_dec") or name.startswith("argmax_dec") or \
                    name in ("gumbel_dec", "gumbel_dec_ws"):
                # Launch-latency-bound: eager timing is the host's launch rate; the graph replay is
                # the device time per launch.
                us_g = time_graph(w, 20, 10) * 1000
                ops[name]["us_graph"] = round(us_g, 3)
                extra = f"  (graph {us_g:.2f} us)"
            log(f"{name:15s} {ms * 1000:10.2f} us  {gbs:8.1f} GB/s  {gbs / PEAK_GBS * 100:5.1f}%  {w.desc}{extra}")

        ms_copy = time_launches(works["calib_copy"], args.steps, args.warmup)
        copy_gbs = works["calib_copy"].nbytes / (ms_copy * 1e-3) / 1e9
        log(f"plain copy 1 GiB: {ms_copy * 1000:.1f} us, {copy_gbs:.1f} GB/s ({copy_gbs / PEAK_GBS * 100:.1f}% of peak)")

        dec = {}
        for name in ("decode_fused", "decode_naive"):
            dec[name] = {"us_eager": ops[name]["us"], "us_graph": round(time_graph(works[name], 20, 10) * 1000, 3)}
        graph = {"fused_us": dec["decode_fused"]["us_graph"], "naive_us": dec["decode_naive"]["us_graph"],
                 "speedup": round(dec["decode_naive"]["us_graph"] / dec["decode_fused"]["us_graph"], 3),
                 "timing": "HIP graph replay of 20 layers x 10 replays"}
        eager_py = {"fused_us": dec["decode_fused"]["us_eager"], "naive_us": dec["decode_naive"]["us_eager"],
                    "speedup": round(dec["decode_naive"]["us_eager"] / dec["decode_fused"]["us_eager"], 3),
                    "timing": "back-to-back launches from Python ctypes"}
        decode = {"graph": graph, "eager_python": eager_py, "eager_compiled": dec_compiled,
                  "desc": "one 64-row decode layer's row ops, f16: 2 residual norms + q/k norm RoPE + SiLU-mul; "
                          "fused (4 launches) vs the naive unfused HIP baseline (10 launches).  The headline "
                          "figures are eager_compiled: back-to-back launches from C++ through the host layer, "
                          "the regime of the reference's batched decode (not graph-captured)"}
        if dec_compiled:
            decode.update({k: dec_compiled[k] for k in ("fused_us", "naive_us", "speedup")})
        log(f"decode layer T=64: eager from C++ x{(dec_compiled or {}).get('speedup')}; graph fused "
            f"{graph['fused_us']:.2f} us vs naive {graph['naive_us']:.2f} us (x{graph['speedup']:.2f}); "
            f"eager from Python x{eager_py['speedup']:.2f}")
        pf, pu = ops["rope_kv_prefill"]["us"], ops["rope_kv_prefill_unfused"]["us"]
        df, du = ops["rope_kv_dec"]["us_graph"], ops["rope_kv_dec_unfused"]["us_graph"]
        rope_kv = {"prefill_4096": {"fused_us": pf, "unfused_us": pu, "speedup": round(pu / pf, 3)},
                   "decode_64x1_graph": {"fused_us": df, "unfused_us": du, "speedup": round(du / df, 3)},
                   "desc": "q/k norm + RoPE + paged KV append: one exl3r_rope_paged_kv launch vs exl3r_rope "
                           "followed by a separate append kernel"}
        log(f"rope + paged KV append: prefill fused {pf:.2f} us vs {pu:.2f} us (x{pu / pf:.2f}); "
            f"decode graph {df:.2f} us vs {du:.2f} us (x{du / df:.2f})")
        c2 = rms_c2_latencies()
        log(f"C2 residual RMSNorm us (graph): {[c2[t]['us_graph'] for t in c2]}")
        sampling = {
            "argmax_64x151936_graph_us": {"exl3r": ops["argmax_dec"]["us_graph"],
                                          "exl3r_one_launch_workspace": ops["argmax_dec_ws"]["us_graph"],
                                          "torch_argmax": ops["argmax_dec_torch"]["us_graph"]},
            "argmax_1024x151936_us": {"exl3r": ops["argmax_prefill"]["us"],
                                      "torch_argmax": ops["argmax_prefill_torch"]["us"]},
            "gumbel_64x151936_us": {"exl3r_graph": ops["gumbel_dec"]["us_graph"],
                                    "exl3r_one_launch_workspace_graph": ops["gumbel_dec_ws"]["us_graph"],
                                    "torch_softmax_multinomial_eager": ops["gumbel_dec_torch"]["us"]},
            "gumbel_1024x151936_us": {"exl3r": ops["gumbel_prefill"]["us"]},
            "desc": "f16 logits; argmax vs torch.argmax (the generator's greedy path); Gumbel-max draw vs "
                    "softmax + multinomial (the reference sampler's tch path)"}
        log(f"sampling: {json.dumps(sampling)}")
        hadamard = {"had_r_128_8192x5120_us": ops["had_c3"]["us"]}
        for fused, label in (("norm_had_c3", "res_norm_to_3_inputs_8192x5120"),
                             ("norm_had_rot_c3", "rotate_res_norm_to_3_inputs_8192x5120"),
                             ("silu_had_c3", "silu_mul_to_input_8192x17408"), ("rope_had_c4", "qk_rotate_rope_c4"),
                             ("rope_kv_had_prefill", "qkv_rotate_rope_paged_append_4096"),
                             ("mlp_had_c3", "rotate_gate_up_silu_mul_to_input_8192x17408"),
                             ("prefill_layer", "qwen3_32b_prefill_layer_T4096"),
                             ("gated_norm_had_q35", "qwen35_gdn_norm_to_o_proj_input_4096x32x128")):
            f_us, u_us = ops[fused]["us"], ops[fused + "_unfused"]["us"]
            hadamard[label] = {"fused_us": f_us, "unfused_us": u_us, "speedup": round(u_us / f_us, 3)}
        hadamard["desc"] = ("the EXL3 linear's random-Hadamard rotation (had_r_128) alone, and fused into the op that "
                            "produces its input or consumes its output, vs the same calls one after another")
        log(f"hadamard: {json.dumps(hadamard)}")
        r_us, c_us, t_us = ops["rope_c4"]["us"], ops["rope_cs_c4"]["us"], ops["rope_cs_table_c4"]["us"]
        rope_cs = {"rope_c4_us": r_us, "rope_cs_c4_us": c_us, "table_per_forward_us": t_us,
                   "per_layer_saving_us": round(r_us - c_us, 2),
                   "paged_append_4096_us": {"evaluated": ops["rope_kv_prefill"]["us"],
                                            "table": ops["rope_kv_prefill_cs"]["us"]},
                   "qkv_rotate_paged_append_4096_us": {"evaluated": ops["rope_kv_had_prefill"]["us"],
                                                       "table": ops["rope_kv_had_prefill_cs"]["us"]},
                   "qwen3_32b_prefill_layer_T4096_us": {"evaluated": ops["prefill_layer"]["us"],
                                                        "table": ops["prefill_layer_cs"]["us"]},
                   "desc": "C4 RoPE evaluating sin / cos in every layer vs reading a {cos, sin} table built once "
                           "per forward pass (bit-identical results); the table costs table_per_forward_us once"}
        log(f"rope_cs: {json.dumps(rope_cs)}")
        qf, qu = ops["qg_rope_q35"]["us"], ops["qg_rope_q35_unfused"]["us"]
        gated_attn = {"fused_us": qf, "unfused_us": qu, "speedup": round(qu / qf, 3),
                      "desc": "Qwen3.5 gated attention's q | g split + q/k head-norm RoPE + output gate, 4096 tokens, "
                              "32/4 heads of 128: rope_qg with the gate read in place vs deinterleave + rope + gate"}
        log(f"gated_attention: {json.dumps(gated_attn)}")

        # The timed step: config-3 prefill row ops back to back (no event between the kernels: an event
        # record between two launches costs the next one a cache flush).
        step_works = [works[n] for n in STEP_OPS]
        step_bytes = sum(w.nbytes for w in step_works)
        for i in range(args.warmup):
            for w in step_works:
                w.launch(i)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(args.steps):
            for w in step_works:
                w.launch(args.warmup + i)
        e.record()
        torch.cuda.synchronize()
        ms_step = s.elapsed_time(e) / args.steps

    value = step_bytes / (ms_step * 1e-3) / 1e9
    # Each step kernel: its HIP-event time over back-to-back launches of it alone (ops above), and its
    # duration inside the step sequence from a rocprofv3 kernel trace of that sequence in this run.  The
    # roofline is quoted on the step's dominant kernel, the one that takes the most time in the step.
    in_step = None if args.no_traffic else trace_step(args.steps, args.warmup)
    kernels = {}
    for n in STEP_OPS:
        v = ops[n]
        kernels[n] = {"kernel": STEP_KERNELS[n], "bytes": v["bytes"], "us": v["us"], "gbs": v["gbs"],
                      "frac": v["frac_peak"]}
        if in_step and n in in_step:
            us = in_step[n]
            kernels[n].update({"us_in_step": round(us, 3), "frac_in_step": round(v["bytes"] / (us * 1e-6) / 1e9 / PEAK_GBS, 4)})
    by = "us_in_step" if in_step and all(n in in_step for n in STEP_OPS) else "us"
    dom_name = max(kernels, key=lambda n: kernels[n][by])
    dom = kernels[dom_name]
    log("C3 step kernels: " + ", ".join(
        f"{n} {v['us']:.2f} us alone" + (f", {v['us_in_step']:.2f} us in the step" if "us_in_step" in v else "")
        for n, v in kernels.items()))
    roof = {"bound": "hbm", "achieved": dom["gbs"], "peak": PEAK_GBS, "unit": "GB/s", "frac": dom["frac"],
            "traffic": None, "kernel": f"{dom['kernel']} ({dom_name})", "bytes_per_launch": dom["bytes"],
            "timing": "HIP events on the launch stream over back-to-back launches of the kernel (us); its "
                      "median duration inside the step sequence from a rocprofv3 kernel trace in this run (us_in_step); "
                      "the dominant kernel is the slowest " + ("in the step" if by == "us_in_step" else "alone"),
            "kernels": kernels}
    if not args.no_traffic:
        t0 = time.time()
        lt = live_traffic(dom_name)
        if lt:
            roof["traffic"] = lt[0]
            roof["traffic_source"] = ("rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on bench.py --op " + dom_name +
                                      " in this run, scaled by the same counters on a 1 GiB copy")
            roof["traffic_detail"] = {"kernel": lt[1], **lt[2],
                                      "traffic_over_algorithmic": round(lt[0] / dom["bytes"], 4)}
        else:
            roof["traffic_source"] = "counter runs unavailable in this run"
        log(f"traffic of {dom_name}: {roof['traffic']} bytes ({time.time() - t0:.0f} s of counter runs)")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['affinity_cores']} in the mask); "
            + ", ".join(f"{k} {v['us']:.0f} us" for k, v in cpu["configs"].items()))
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded N(0,1) activations, N(0,4) residual, N(1,0.1) weights, N(0,0.02) table, "
                "Zipf(1.1) ids, ragged positions",
        "config": {"workload": "C3 prefill row ops (BASELINE configs[2]): residual RMSNorm [8192,5120] + "
                               "SiLU-mul + GELU-mul [8192,17408], bf16 I/O, fp32 arithmetic",
                   "io_dtype": "bf16", "tokens": 8192, "hidden": 5120, "intermediate": 17408,
                   "frac_peak": round(value / PEAK_GBS, 4)},
        "roofline": roof, "cpu_baseline": cpu, "ops": ops, "decode_step": decode, "c2_decode_rms_norm": c2,
        "rope_paged_kv": rope_kv, "sampling": sampling, "hadamard": hadamard, "rope_cs_table": rope_cs,
        "gated_attention_qg": gated_attn,
        "copy_reference": {"gbs": round(copy_gbs, 1), "frac_peak": round(copy_gbs / PEAK_GBS, 4),
                           "desc": "non-temporal 16 B/lane device copy of 1 GiB (read + write), the practical HBM ceiling reference"},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
