"""Salient-path throughput of one sparse denoise step at the LLaDA-8B shape (config 1).

Workload (one MI355X): 32 layers, hidden 4096, 32 heads x 128,
SwiGLU 12288, batch 8 x 1024 rows (256 prompt + 768 response), tau = 0.99, a Q-pruned sparse
step. Random-init bf16 weights N(0, 0.02); K/V/Q ~ N(0, 1). The caches hold a dense
"step 1" (our dense attention); 15% of the response rows of every sequence are perturbed in
the cached context with Gaussian noise of 0.5 x row RMS and get fresh K/V rows, which makes
~15% of the rows salient at every layer, as in the reference's synthetic recipe.

One step = for every layer: RoPE + K-cache scatter of the salient rows' projected keys (the
fused K/V epilogue), dV + V-cache update,
row-sparse attention of the salient queries vs the full cached K/V, column-sparse attention
with the saliency statistics and the tau test, compaction of the next salient set (one host
read of its size, as the reference's torch.nonzero), gathered SwiGLU GEMMs with the
scatter into the FFN cache. The queried FFN rows are left in the FFN cache, where the next
layer's residual + RMSNorm reads them in place (ops.CacheRows), as in the model. The dense
projections/norms on either side of the path are outside the timed region (their inputs are
pre-generated per layer). The caches are restored between steps (untimed) so every timed
step sees the same salient fraction.

Steps follow config 1's cadence: step i of the timed K is a refresh step (every row queried,
T = 8192, the salient set in K space) when i % 4 == 3, and a Q-pruned step (the 6144 response
rows) otherwise; both denoise the same B * Lq = 6144 answer tokens.

value = B * Lq / mean step time over the K steps (tokens/s); the Q-pruned and refresh steps are
also reported on their own. The roofline object is for the dominant kernel of the Q-pruned step,
the fused attention kernel (timed with library-owned HIP events around that launch,
dyllm_attention_timer) or the gathered gate_up SwiGLU GEMM (HIP events on its own launches),
whichever has the longer mean launch; the other rides along, as do the down GEMM, the fused
kernel of the refresh step, the dense full-step attention, config 3's MoE expert FFN and the
salient-row K/V projection (the step before the path, outside `value`), each timed with HIP
events on its launching stream.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

CONFIG1 = dict(layers=32, hidden=4096, heads=32, kv_heads=32, head_dim=128, inter=12288, batch=8, prompt=256,
               response=768, tau=0.99, perturb=0.15)
# BASELINE.json configs[2] (Dream-v0-7B shape, GQA 28/4, perturbed fraction 25 % of {5, 25, 50} %) and
# configs[4] (LLaDA-8B shape at 8192 rows per sequence, tau 0.995, refresh every 8 steps)
CONFIG2 = dict(layers=28, hidden=3584, heads=28, kv_heads=4, head_dim=128, inter=18944, batch=16, prompt=512,
               response=1536, tau=0.99, perturb=0.25)
CONFIG4 = dict(layers=32, hidden=4096, heads=32, kv_heads=32, head_dim=128, inter=12288, batch=2, prompt=2048,
               response=6144, tau=0.995, perturb=0.05)
PEAK_BF16_TFLOPS = 2500.0
EVENT_STRIDE = 8
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of the gate_up GEMM at this workload, from rocprofv3 FETCH_SIZE / WRITE_SIZE
# calibrated against a 256 MiB copy (profiles/pmc_gemm_gate_up_config1.md).
GATE_UP_TRAFFIC_BYTES = 345.0e6
# HBM bytes per launch of the fused attention kernel, same method (profiles/pmc_attention_step_config1.md)
ATTN_TRAFFIC_BYTES = 418.9e6


def build_workload(cfg, layers, device, seed=0):
    import torch

    from dyllm_amd import _lib, ops
    from dyllm_amd.engine.cache_manager import CacheManager
    from dyllm_amd.model_executor.layers.attention import Attention
    from dyllm_amd.model_executor.models.llada import LLaDAMLP
    from dyllm_amd.utils.context import set_context
    from dyllm_amd.utils.metadata import get_metadata

    B, P, R = cfg["batch"], cfg["prompt"], cfg["response"]
    L = P + R
    H, Hkv, D, hid, inter = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["hidden"], cfg["inter"]
    Tk, Tq = B * L, B * R
    g = torch.Generator(device=device).manual_seed(seed)
    gcpu = torch.Generator().manual_seed(seed)
    md = get_metadata()
    md.running_seqs = list(range(B))
    md.running_seqs_tensor = torch.arange(B, dtype=torch.long, device=device)
    md.finished_seqs = []
    cu_k_cpu = [i * L for i in range(B + 1)]
    cu_q_cpu = [i * R for i in range(B + 1)]
    cu_p_cpu = [i * P for i in range(B + 1)]
    i32 = dict(dtype=torch.int32, device=device)
    cu_k, cu_q, cu_p = (torch.tensor(x, **i32) for x in (cu_k_cpu, cu_q_cpu, cu_p_cpu))

    # salient rows: the same 15% of each sequence's response rows at every layer
    n_per = int(round(cfg["perturb"] * R))
    sq, sk = [], []
    for b in range(B):
        sel = torch.randperm(R, generator=gcpu)[:n_per].sort().values
        sq += (b * R + sel).tolist()
        sk += (b * L + P + sel).tolist()
    S_q = torch.tensor(sq, dtype=torch.long, device=device)
    S_k = torch.tensor(sk, dtype=torch.long, device=device)
    cu_s = torch.tensor([i * n_per for i in range(B + 1)], **i32)

    def randn(*shape, std=1.0):
        x = torch.empty(*shape, dtype=torch.float32, device=device)
        x.normal_(0.0, std, generator=g)
        return x.to(torch.bfloat16)

    state = []
    for _ in range(layers):
        # dense "step 1": fill K, V and context caches (attention.py:39-62)
        set_context(True, cu_seqlens_q=cu_k, cu_seqlens_q_cpu=cu_k_cpu, cu_seqlens_k=cu_k,
                    cu_seqlens_k_cpu=cu_k_cpu, max_seqlen_q=L, max_seqlen_k=L, context_lens_cpu=[L] * B,
                    total_seqlen=Tk, total_seqlen_k=Tk)
        attn = Attention(H, D, D ** -0.5, Hkv, cfg["tau"], device=device)
        k_cache = CacheManager(Hkv * D, device=torch.device(device))
        mlp = LLaDAMLP(hid, inter, device=device, gen=g)
        attn.ffn_cache = mlp.cache_update.cache_manager   # the step computes the FFN's scatter rows
        q_all, k_all, v_all = randn(Tk, H, D), randn(Tk, Hkv, D), randn(Tk, Hkv, D)
        k_cache.reset_full(k_all.view(Tk, -1), md.running_seqs_tensor, md.running_seqs)
        attn(q_all, k_all, v_all)
        mlp.cache_update(randn(Tk, hid))
        # perturb the cached context of the salient rows (sigma = 0.5 x row RMS)
        c = attn.context_cache.cache
        rows = c[S_k].float()
        rms = rows.pow(2).mean(-1, keepdim=True).sqrt()
        c[S_k] = (rows + 0.5 * rms * randn(len(sk), H * D).float()).to(torch.bfloat16)
        resp = torch.cat([torch.arange(b * L + P, (b + 1) * L, device=device) for b in range(B)])
        q = q_all[resp].contiguous()
        q_full = q_all     # the refresh step queries every row
        # stand-in for the salient-row K/V projection output: kv rows [k | v] of every K row
        # (addressed by K-space salient index in both step kinds, so any salient set is in range)
        k_new = (k_all.float() + 0.1 * randn(Tk, Hkv, D).float()).to(torch.bfloat16)
        v_new = (v_all.float() + 0.1 * randn(Tk, Hkv, D).float()).to(torch.bfloat16)
        del k_all, v_all
        kv_all = torch.cat([k_new.view(Tk, -1), v_new.view(Tk, -1)], dim=1).contiguous()
        del k_new, v_new
        state.append(dict(attn=attn, k_cache=k_cache, mlp=mlp, q=q, q_full=q_full, kv_all=kv_all,
                          c_saved=attn.context_cache.cache.clone(), v_saved=attn.v_cache.cache.clone()))
    torch.cuda.synchronize()
    # RoPE tables (rotary_embedding.py:19-38, theta 500000); every position 0, where the rotation
    # is the identity, so the fused epilogue does its full work without changing the keys
    # (and with them the salient fraction the workload is built for)
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32, device=device) / D))
    freqs = torch.outer(torch.arange(4096, dtype=torch.float32, device=device), inv)
    rope_cos, rope_sin = freqs.cos().contiguous(), freqs.sin().contiguous()
    pos0 = torch.zeros(Tk, dtype=torch.long, device=device)

    def set_sparse_context(refresh):
        if refresh:   # every row queried; the salient set lives in K space (model_runner.py:217-222)
            return set_context(False, cu_seqlens_q=cu_k, cu_seqlens_q_cpu=cu_k_cpu, cu_seqlens_k=cu_k,
                               cu_seqlens_k_cpu=cu_k_cpu, cu_promptlens=cu_p, max_seqlen_q=L, max_seqlen_k=L,
                               context_lens_cpu=[L] * B, cu_salientlens=cu_s, idx_salient_row=S_k,
                               idx_salient_row_i32=S_k.to(torch.int32), idx_salient_row_k=None,
                               max_salientlen=n_per, total_seqlen=Tk, total_seqlen_k=Tk)
        return set_context(False, cu_seqlens_q=cu_q, cu_seqlens_q_cpu=cu_q_cpu, cu_seqlens_k=cu_k,
                           cu_seqlens_k_cpu=cu_k_cpu, cu_promptlens=cu_p, max_seqlen_q=R, max_seqlen_k=L,
                           context_lens_cpu=[L] * B, cu_salientlens=cu_s, idx_salient_row=S_q,
                           idx_salient_row_i32=S_q.to(torch.int32), idx_salient_row_k=S_k, max_salientlen=n_per,
                           total_seqlen=Tq, total_seqlen_k=Tk)

    def restore():
        for st in state:
            st["attn"].context_cache.cache.copy_(st["c_saved"])
            st["attn"].v_cache.cache.copy_(st["v_saved"])

    kv_proj = {}

    def step(events=None, n_sal=None, refresh=False, with_kv_proj=False):
        ctx = set_sparse_context(refresh)
        T = Tk if refresh else Tq
        if with_kv_proj and not kv_proj:
            # salient-row K/V projection operands: layer inputs of every K row and 4 weight copies
            # cycled over the layers (so the weights come from HBM, as across 32 layers)
            kv_proj["x"] = randn(Tk, hid)
            kv_proj["w"] = [randn(2 * Hkv * D, hid, std=0.02) for _ in range(4)]
        for li, st in enumerate(state):
            idx = ctx.idx_salient_row
            if n_sal is not None:
                n_sal.append(idx.numel())
            if with_kv_proj:
                # the projection GEMM of the salient rows (dyllm_linear, llada.py:108); its output
                # is not consumed: the epilogue below keeps the stand-in rows, so the salient fraction
                # of the workload stays as built
                ops.linear(kv_proj["x"], kv_proj["w"][li % 4], rows_idx=ctx.idx_salient_row_i32)
            # the projection's [k | v] rows of the salient set (stand-in: rows of pre-generated
            # [k | v] addressed by K-space index); the step's first launch applies their epilogue
            # (RoPE + K-cache row of k) and takes v from them
            kidx32 = ctx.idx_salient_row_i32 if refresh else ctx.idx_salient_row_k_i32
            v_sal = st["k_cache"].kv_rows(st["kv_all"], Hkv, pos0, rope_cos, rope_sin, ctx.idx_salient_row_i32,
                                          kv_rows=kidx32)
            ev = events.get(li) if events is not None else None
            if ev is not None:   # time the fused attention kernel of this layer's step call
                _lib.load().dyllm_attention_timer(1)
            o = st["attn"](st["q_full"] if refresh else st["q"], None, v_sal)
            if ev is not None:
                _lib.load().dyllm_attention_timer(0)
            # the FFN rows stay in the FFN cache (the next layer's norm reads them in place)
            st["mlp"].forward_salient(o.view(T, H * D), timing=ev, lazy=True)
        return ctx

    return dict(step=step, restore=restore, Tq=Tq, Tk=Tk, n_per=n_per, S_q=S_q, state=state)


def _median_time(fn, warmup=2, repeats=5):
    """2 warm-ups, then the median of `repeats` wall-clock runs (time.perf_counter)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def _cpu_layer(ref, torch, np, B, P, R, H, Hkv, D, hid, inter, n_per, tau, seed):
    """Inputs of one sparse layer of the saliency path for the CPU oracle, and the closure that
    runs it: RoPE of the salient keys, row-sparse attention of the salient queries, column-sparse
    attention + statistics + tau test, compaction + fused offset, gathered SwiGLU FFN."""
    L = P + R
    Tk, Tq = B * L, B * R
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    q = torch.randn(Tq, H, D, generator=g).to(bf)
    k = torch.randn(Tk, Hkv, D, generator=g).to(bf)
    v = torch.randn(Tk, Hkv, D, generator=g).to(bf)
    c = torch.randn(Tq, H, D, generator=g).to(bf)
    rng = np.random.default_rng(seed)
    idx_q, idx_k = [], []
    for b in range(B):
        sel = np.sort(rng.choice(R, size=n_per, replace=False))
        idx_q += (b * R + sel).tolist()
        idx_k += (b * L + P + sel).tolist()
    idx_q, idx_k = np.asarray(idx_q), np.asarray(idx_k)
    cu_q, cu_k, cu_p, cu_s = (np.arange(B + 1) * x for x in (R, L, P, n_per))
    dv = torch.zeros_like(k)
    dv[idx_k] = (0.1 * torch.randn(len(idx_k), Hkv, D, generator=g)).to(bf)
    w_gu = (0.02 * torch.randn(2 * inter, hid, generator=g)).to(bf)
    w_d = (0.02 * torch.randn(hid, inter, generator=g)).to(bf)
    rope_cos, rope_sin = ref.rope_tables(D, 4096, 500000.0)
    ik, iq = torch.from_numpy(idx_k), torch.from_numpy(idx_q)
    pos = torch.zeros(len(idx_k), dtype=torch.long)

    def run():
        kk = k.clone()
        kk[ik] = ref.rope_neox(kk[ik], rope_cos, rope_sin, pos)
        o_sal = ref.flash_attn_varlen(q[iq], kk, v, cu_s, cu_k)
        new_c, _, mask = ref.attention_sparse_varlen(q, kk, dv, c, o_sal, cu_q, cu_k, idx_q, tau)
        idxs, cu_sal = ref.compact(mask.numpy(), cu_q)
        ref.fused_offset(idxs, cu_p, cu_sal)
        ref.swiglu_ffn(new_c.reshape(Tq, -1)[iq], w_gu, w_d)

    return run


def cpu_baseline(cfg, n_sal, threads):
    """The CPU oracle (fp32 torch / numpy restatement of the reference path) on the GPU box's host,
    timed as 2 warm-ups + the median of 5 repeats: one config-1 layer at full shape (x the layer
    count), and config 0 (one layer, B = 1, 128 + 384 rows, 10 % salient) in full."""
    import numpy as np
    import torch

    from oracle import dyllm_oracle as ref

    torch.set_num_threads(threads)
    B, P, R = cfg["batch"], cfg["prompt"], cfg["response"]
    H, Hkv, D, hid, inter = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["hidden"], cfg["inter"]
    n_per = max(1, n_sal // B)
    run1 = _cpu_layer(ref, torch, np, B, P, R, H, Hkv, D, hid, inter, n_per, cfg["tau"], 1)
    t_layer = _median_time(run1)
    run0 = _cpu_layer(ref, torch, np, 1, 128, 384, 32, 32, 128, 4096, 12288, 38, cfg["tau"], 2)
    t0 = _median_time(run0)
    Tq = B * R
    return dict(value=Tq / (t_layer * cfg["layers"]), unit="tokens/s", cores=threads, kind="port",
                sample=f"1 of {cfg['layers']} layers at full config-1 shape ({n_per * B} salient rows): "
                       f"median {t_layer:.3f} s of 5 after 2 warm-ups, x{cfg['layers']} layers",
                config0={"value": 384 / t0, "unit": "tokens/s", "ms_per_layer": round(t0 * 1e3, 2),
                         "sample": "config 0 in full: one layer, B=1, 128+384 rows, 38 salient rows, "
                                   "median of 5 after 2 warm-ups"})


def time_kv_projection(cfg, n_sal, reps=24, copies=8):
    """The salient-row K/V projection (dyllm_linear: kv = hidden[idx] . W_kv^T, llada.py:108) at
    the bench shape, timed with HIP events on the launching stream, cycling through `copies`
    weight matrices so the weights come from HBM as they do across 32 layers."""
    import torch

    from dyllm_amd import _lib, ops

    dev = "cuda"
    hid, kv_out = cfg["hidden"], 2 * cfg["kv_heads"] * cfg["head_dim"]
    Tq = cfg["batch"] * cfg["response"]
    g = torch.Generator(device=dev).manual_seed(1)
    ws = [torch.empty(kv_out, hid, device=dev).normal_(0, 0.02, generator=g).to(torch.bfloat16)
          for _ in range(copies)]
    x = torch.empty(Tq, hid, device=dev).normal_(generator=g).to(torch.bfloat16)
    rows = torch.sort(torch.randperm(Tq, device=dev, generator=g)[:n_sal]).values.to(torch.int32)
    for w in ws:
        ops.linear(x, w, rows_idx=rows)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for i, (e0, e1) in enumerate(evs):
        e0.record()
        ops.linear(x, ws[i % copies], rows_idx=rows)
        e1.record()
    torch.cuda.synchronize()
    us = sum(e0.elapsed_time(e1) for e0, e1 in evs) / reps * 1e3
    flops = 2.0 * n_sal * hid * kv_out
    tf = flops / (us * 1e-6) / 1e12
    bm = _lib.load().dyllm_ffn_tile_rows(n_sal, kv_out, hid, 0)
    return {"kernel": f"gemm_kernel<{bm},4,Store> (dyllm_linear: gathered kv_proj of the salient rows)",
            "rows": n_sal, "avg_launch_us": round(us, 2), "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "flop_per_launch": flops}


def profile_hbm(cfg, reps=5):
    """The HBM-bound kernels of the path as standalone launches at the config-1 shape (6144
    queried rows x 4096, 15 % salient): saliency statistics + tau test, compaction, gather,
    scatter into a cache, FFN-cache read-back (get_block), fused residual + RMSNorm and the K/V
    epilogue. Each runs `reps` times back to back; HIP events on the launching stream give the
    per-launch time, printed with the algorithmic bytes and the fraction of the 8 TB/s peak (run
    under rocprofv3 --kernel-trace --stats for the profiler's own durations)."""
    import torch

    from dyllm_amd import ops

    dev = "cuda"
    B, P, R, hid = cfg["batch"], cfg["prompt"], cfg["response"], cfg["hidden"]
    L, Tq = P + R, B * R
    Hkv = cfg["kv_heads"]
    kvs = Hkv * cfg["head_dim"]
    n_per = int(round(cfg["perturb"] * R))
    g = torch.Generator(device=dev).manual_seed(2)
    bf = torch.bfloat16

    def randn(*shape):
        return torch.empty(*shape, device=dev).normal_(generator=g).to(bf)

    c_old = randn(Tq, hid)
    c_new = c_old.clone()
    sel = torch.cat([b * R + torch.randperm(R, device=dev, generator=g)[:n_per].sort().values for b in range(B)])
    c_new[sel] = randn(len(sel), hid)
    n_sal = len(sel)
    i32 = dict(dtype=torch.int32, device=dev)
    cu_q = torch.arange(B + 1, **i32) * R
    cu_k = torch.arange(B + 1, **i32) * L
    cu_p = torch.arange(B + 1, **i32) * P
    seq_ids = torch.arange(B, dtype=torch.long, device=dev)
    starts = torch.arange(B, dtype=torch.long, device=dev) * L
    cache = randn(B * L, hid)
    idx_k = (sel // R) * L + P + sel % R
    x = randn(Tq, hid)
    resid = randn(Tq, hid)
    w = torch.ones(hid, dtype=bf, device=dev)
    kv = randn(n_sal, 2 * kvs)
    k_cache = randn(B * L, kvs)
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32, device=dev) / 128))
    fr = torch.outer(torch.arange(4096, dtype=torch.float32, device=dev), inv)
    cos, sin = fr.cos().contiguous(), fr.sin().contiguous()
    positions = torch.arange(Tq, dtype=torch.long, device=dev)
    stats, mask = ops.saliency_stats(c_new, c_old, cfg["tau"])
    row = hid * 2
    cases = [
        ("saliency_rows_kernel (stats + tau test)", lambda: ops.saliency_stats(c_new, c_old, cfg["tau"]),
         Tq * (2 * row + 13)),
        ("compact_kernel (salient index lists)", lambda: ops.salient_compact(mask, cu_q, cu_p),
         Tq + n_sal * 20 + 4 * (B + 1)),
        ("row_map_copy_kernel<Gather> (salient rows)", lambda: ops.gather_rows_2D(x, sel), n_sal * 2 * row),
        ("row_map_copy_kernel<Scatter> (rows into a cache)",
         lambda: ops.scatter_update_cuda(cache, c_new[:n_sal], idx_k, cu_k, starts, seq_ids), n_sal * 2 * row),
        ("row_map_copy_kernel<GetBlock> (queried rows back)",
         lambda: ops.get_block_cuda(cache, starts, cu_k, cu_q, seq_ids, Tq), Tq * 2 * row),
        ("add_rms_norm_kernel (residual + RMSNorm)", lambda: ops.rms_norm(x, w, 1e-6, residual=resid), Tq * 4 * row),
        ("kv_rope_scatter_kernel (RoPE + K-cache rows + V)",
         lambda: ops.kv_rope_scatter(kv, Hkv, positions, cos, sin, k_cache, idx_k, cu_k, starts, seq_ids,
                                     pos_idx=sel), n_sal * 4 * kvs * 2),
    ]
    sel32 = sel.to(torch.int32)
    cases[-1] = (cases[-1][0], lambda: ops.kv_rope_scatter(kv, Hkv, positions, cos, sin, k_cache, idx_k, cu_k, starts,
                                                           seq_ids, pos_idx=sel32), cases[-1][2])
    # size references: the same gather over every queried row, and torch's contiguous device copy
    # of the salient-row bytes and of the full-size bytes (what one launch of that size reaches)
    all_rows = torch.randperm(Tq, device=dev, generator=g)
    src_s, dst_s = randn(n_sal, hid), randn(n_sal, hid)
    src_f, dst_f = randn(Tq, hid), randn(Tq, hid)
    cases += [
        ("row_map_copy_kernel<Gather> (every queried row, permuted)", lambda: ops.gather_rows_2D(x, all_rows),
         Tq * 2 * row),
        ("reference: torch copy_ of the salient-row bytes", lambda: dst_s.copy_(src_s), n_sal * 2 * row),
        ("reference: torch copy_ of the queried-row bytes", lambda: dst_f.copy_(src_f), Tq * 2 * row),
    ]
    print("| kernel | algorithmic bytes per launch | us per launch (HIP events, back to back) | GB/s | of 8 TB/s |")
    print("|---|---:|---:|---:|---:|")
    for name, fn, nbytes in cases:
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        # launches of a few us are bounded by the host's enqueue rate here; the profiler's
        # per-kernel durations are the reference for those
        us = e0.elapsed_time(e1) / reps * 1e3
        gbs = nbytes / (us * 1e-6) / 1e9
        print(f"| `{name}` | {nbytes / 1e6:.2f} MB | {us:.1f} | {gbs:.0f} | {gbs / PEAK_HBM_GBS:.0%} |", flush=True)


def profile_gate_up(cfg, reps=3):
    """Counter-collection workload: the gathered gate_up GEMM at the bench shape (15% of the
    response rows salient) interleaved with a 256 MiB device copy used to calibrate the HBM
    byte counters. Run under rocprofv3 --pmc."""
    import torch

    from dyllm_amd import ops

    dev = "cuda"
    hid, inter = cfg["hidden"], cfg["inter"]
    Tq = cfg["batch"] * cfg["response"]
    M = int(round(cfg["perturb"] * cfg["response"])) * cfg["batch"]
    g = torch.Generator(device=dev).manual_seed(0)
    w = torch.empty(2 * inter, hid, device=dev).normal_(0, 0.02, generator=g).to(torch.bfloat16)
    x = torch.empty(Tq, hid, device=dev).normal_(generator=g).to(torch.bfloat16)
    rows = torch.sort(torch.randperm(Tq, device=dev, generator=g)[:M]).values.to(torch.int32)
    a = torch.empty(128 * 1024 * 1024, dtype=torch.bfloat16, device=dev).normal_(generator=g)
    b = torch.empty_like(a)
    for _ in range(reps):
        ops.ffn_gate_up(x, w, rows)
        b.copy_(a)  # calibration: 256 MiB read + 256 MiB written
    # the gather's and the scatter's share: the same products on contiguous rows, in this order
    # (dispatches in the counter file follow it): gate_up gathered, gate_up contiguous, down with
    # the FFN-cache scatter (random cache rows), down contiguous
    xc = x[rows.long()].contiguous()
    wd = torch.empty(hid, inter, device=dev).normal_(0, 0.02, generator=g).to(torch.bfloat16)
    cache = torch.empty(cfg["batch"] * (cfg["prompt"] + cfg["response"]), hid, dtype=torch.bfloat16, device=dev)
    dest = torch.randperm(cache.shape[0], device=dev, generator=g)[:M]
    h = ops.ffn_gate_up(xc, w)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(4)]
    cases = [lambda: ops.ffn_gate_up(x, w, rows), lambda: ops.ffn_gate_up(xc, w),
             lambda: ops.ffn_down(h, wd, out=cache, out_rows=dest), lambda: ops.ffn_down(h, wd)]
    ms = [0.0] * 4
    for i, fn in enumerate(cases):
        for _ in range(2):   # warm
            fn()
        for _ in range(reps):
            ev[i][0].record()
            fn()
            ev[i][1].record()
            torch.cuda.synchronize()
            ms[i] += ev[i][0].elapsed_time(ev[i][1]) / reps
    print(f"[bench] profiled gate_up: {reps} launches of M={M}, plus {reps} calibration copies of 256 MiB; then "
          f"{reps} each of gate_up gathered / contiguous and down scattered / contiguous: "
          + ", ".join(f"{v * 1e3:.1f} us" for v in ms), file=sys.stderr)


def profile_attention(cfg, reps=5):
    """Counter-collection workload for the two tile kinds of the fused attention kernel, each as
    its standalone launch at the config-1 Q-pruned shape (6144 queried rows of 8 x 1024 keys, 15 %
    salient): the row-sparse tiles (attention_kernel<RowSparse>: the salient queries against all
    keys and the updated V) and the two-pass column-sparse tiles (attention_kernel<ColSparse,4>:
    QK^T and the row statistics over all keys, PV over the salient keys' dV). Prints the HIP-event
    time of each; run under rocprofv3 --pmc for the instruction and cycle counters."""
    import torch

    from dyllm_amd import ops

    dev = "cuda"
    B, P, R = cfg["batch"], cfg["prompt"], cfg["response"]
    L = P + R
    H, Hkv, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    Tq, Tk = B * R, B * L
    n_per = int(round(cfg["perturb"] * R))
    g = torch.Generator(device=dev).manual_seed(4)
    gcpu = torch.Generator().manual_seed(4)
    rnd = lambda *sh, std=1.0: torch.empty(*sh, device=dev).normal_(0.0, std, generator=g).to(torch.bfloat16)
    q, k, v, c = rnd(Tq, H, D), rnd(Tk, Hkv, D), rnd(Tk, Hkv, D), rnd(Tq, H, D)
    sq, sk = [], []
    for b in range(B):
        sel = torch.randperm(R, generator=gcpu)[:n_per].sort().values
        sq += (b * R + sel).tolist()
        sk += (b * L + P + sel).tolist()
    idx_q = torch.tensor(sq, dtype=torch.int32, device=dev)
    idx_k = torch.tensor(sk, dtype=torch.int32, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    cu_q = torch.arange(B + 1, **i32) * R
    cu_k = torch.arange(B + 1, **i32) * L
    cu_s = torch.arange(B + 1, **i32) * n_per
    dv = rnd(len(sk), Hkv, D, std=0.1)

    def rowsparse():
        return ops.flash_attn_varlen_func(q, k, v, cu_s, cu_k, n_per, L, q_rows=idx_q)

    o_sal = rowsparse()

    def colsparse():
        ops.attention_colsparse_cached(q, k, None, dv, c, None, o_sal, cu_q, cu_k, R, L, Tk, idx_q, idx_k,
                                       cfg["tau"], c_inplace=False)

    colsparse()
    torch.cuda.synchronize()
    out = {}
    for name, fn in (("row-sparse tiles", rowsparse), ("column-sparse tiles", colsparse)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(e0.elapsed_time(e1) / reps * 1e3, 2)
    print(f"[bench] standalone attention tiles at the config-1 Q-pruned shape ({len(sk)} salient rows), "
          f"us per launch: {out}", file=sys.stderr)


def time_dense_attention(cfg, reps=5):
    """Dense full-sequence attention (the full steps, attention.py:39-62: attention_kernel<Dense>)
    at the config-1 shape, T = 8192 rows, HIP events on the launching stream."""
    import torch

    from dyllm_amd import ops

    dev = "cuda"
    B, L = cfg["batch"], cfg["prompt"] + cfg["response"]
    H, Hkv, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    g = torch.Generator(device=dev).manual_seed(3)
    rnd = lambda *sh: torch.empty(*sh, device=dev).normal_(generator=g).to(torch.bfloat16)
    q, k, v = rnd(B * L, H, D), rnd(B * L, Hkv, D), rnd(B * L, Hkv, D)
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev) * L
    ops.flash_attn_varlen_func(q, k, v, cu, cu, L, L)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        ops.flash_attn_varlen_func(q, k, v, cu, cu, L, L)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / reps * 1e3
    flops = 4.0 * B * L * L * H * D
    tf = flops / (us * 1e-6) / 1e12
    return {"kernel": "attention_kernel<Dense,4> (full step, 8 x 1024 rows)", "bound": "mfma",
            "avg_launch_us": round(us, 2), "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / PEAK_BF16_TFLOPS, 4), "flop_per_launch": flops, "traffic": None}


def time_moe(reps=6, copies=4):
    """Config 3's MoE FFN over its salient rows (LLaDA-MoE: hidden 2048, 64 experts, top-8, expert
    SwiGLU 1024; 15 % of 32 x 768 rows salient; router logits ~ N(0, 1) plus a per-expert bias
    ~ N(0, 0.5), carried by a constant input feature, for a skewed load). Times dyllm_fused_experts
    (align + grouped gate_up GEMM + grouped down GEMM + combine) with HIP events, cycling through
    `copies` expert weight sets so the weights come from HBM as across 16 layers."""
    import torch

    from dyllm_amd import ops

    dev = "cuda"
    hid, E, top_k, inter = 2048, 64, 8, 1024
    n = int(round(0.15 * 32 * 768))
    g = torch.Generator(device=dev).manual_seed(5)
    rnd = lambda *sh, std=1.0: torch.empty(*sh, device=dev).normal_(0.0, std, generator=g).to(torch.bfloat16)
    x = rnd(n, hid)
    wr = rnd(E, hid, std=hid ** -0.5)
    x[:, 0] = 1.0
    wr[:, 0] = rnd(E, std=0.5)
    w1s = [rnd(E, 2 * inter, hid, std=hid ** -0.5) for _ in range(copies)]
    w2s = [rnd(E, hid, inter, std=inter ** -0.5) for _ in range(copies)]
    w, ids = ops.moe_gate(x, wr, top_k)
    for i in range(copies):
        ops.fused_experts(x, w1s[i], w2s[i], w, ids)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for i, (e0, e1) in enumerate(evs):
        e0.record()
        ops.fused_experts(x, w1s[i % copies], w2s[i % copies], w, ids)
        e1.record()
    torch.cuda.synchronize()
    us = sum(e0.elapsed_time(e1) for e0, e1 in evs) / reps * 1e3
    # the router (moe_gate: fp32 logits, softmax, top-k) of the same rows, timed on its own
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record()
    for _ in range(reps):
        ops.moe_gate(x, wr, top_k)
    r1.record()
    torch.cuda.synchronize()
    router_us = r0.elapsed_time(r1) / reps * 1e3
    flops = 6.0 * n * top_k * hid * inter
    tf = flops / (us * 1e-6) / 1e12
    load = torch.bincount(ids.reshape(-1).long(), minlength=E)
    return {"kernel": "dyllm_fused_experts (align + grouped gate_up/down gemm_kernel + combine), config 3",
            "bound": "mfma", "rows": n, "slots": n * top_k, "max_expert_load": int(load.max()),
            "mean_expert_load": round(float(load.float().mean()), 1), "avg_launch_us": round(us, 2),
            "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / PEAK_BF16_TFLOPS, 4), "flop_per_launch": flops, "traffic": None,
            "router_us": round(router_us, 2)}


def probe_issue(iters=4096):
    """dyllm_issue_probe at one wavefront per SIMD (256 workgroups of 256 threads): mean cycles per
    loop iteration of 4 MFMA 32x32x16, of 64 FMA, of 64 exp + 64 mul, and of the MFMA loop fused
    with each VALU loop in one wavefront (compiler-scheduled and pinned 1 MFMA : 16 VALU). The
    overlap of MFMA and VALU work = (MFMA + VALU - both) / min(MFMA, VALU)."""
    import torch

    from dyllm_amd import _lib

    wgs = 256
    sink = torch.empty(wgs * 256, dtype=torch.float32, device="cuda")
    cyc = torch.empty(wgs, dtype=torch.int64, device="cuda")
    names = ["mfma", "fma", "exp", "mfma+fma", "mfma+fma pinned", "mfma+exp", "mfma+exp pinned"]
    res = {}
    for mode, name in enumerate(names):
        for _ in range(2):   # the second launch is timed
            _lib.call("dyllm_issue_probe", mode, wgs, iters, sink.data_ptr(), cyc.data_ptr(),
                      torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        res[name] = round(float(cyc.double().mean()) / iters, 1)
    ov = {}
    for both, valu in (("mfma+fma", "fma"), ("mfma+fma pinned", "fma"), ("mfma+exp", "exp"),
                       ("mfma+exp pinned", "exp")):
        ov[both] = round((res["mfma"] + res[valu] - res[both]) / min(res["mfma"], res[valu]), 3)
    print(json.dumps({"probe": "MFMA/VALU issue of one wavefront per SIMD", "cycles_per_iteration": res,
                      "overlap_fraction": ov, "iters": iters, "workgroups": wgs}))


def _attn_flops(T, L, HD, n, n_seq_sal):
    """Algorithmic MFMA work of the fused attention kernel: row-sparse tiles 4 Lk H D per salient
    query row; column-sparse tiles QK^T 2 Lk H D per other row plus PV over the salient keys of
    its sequence."""
    return 4.0 * L * HD * n + 2.0 * L * HD * (T - n) + 2.0 * n_seq_sal * HD * (T - n)


def _read_attn_timer():
    import ctypes

    from dyllm_amd import _lib
    ms, n = ctypes.c_float(), ctypes.c_int()
    _lib.call("dyllm_attention_timer_read", ctypes.addressof(ms), ctypes.addressof(n))
    return ms.value, n.value


def _run_cadence(wl, steps, period, layers, with_kv_proj=False):
    """Timed denoise steps of a built workload: step i is a refresh step when i % period ==
    period - 1, a Q-pruned step otherwise. Per step kind: wall times, salient rows per layer, the
    fused attention launches (library HIP events) and the gate_up / down launches (HIP events on
    every EVENT_STRIDE-th layer)."""
    import torch

    _read_attn_timer()
    kinds = {False: dict(ms=[], attn=[0.0, 0], gate=[], down=[], n_sal=[]),
             True: dict(ms=[], attn=[0.0, 0], gate=[], down=[], n_sal=[])}
    for i in range(steps):
        refresh = i % period == period - 1
        k = kinds[refresh]
        wl["restore"]()
        # GEMM launches are bracketed with HIP events on every EVENT_STRIDE-th layer: each event
        # pair is a pair of marker packets on the stream, so bracketing all layers would add their
        # cost to the measured step
        evs = {li: {"gate_up": (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)),
                    "down": (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))}
               for li in range(0, layers, EVENT_STRIDE)}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        wl["step"](events=evs, n_sal=k["n_sal"], refresh=refresh, with_kv_proj=with_kv_proj)
        torch.cuda.synchronize()
        k["ms"].append((time.perf_counter() - t0) * 1e3)
        k["gate"] += [e["gate_up"][0].elapsed_time(e["gate_up"][1]) for e in evs.values()]
        k["down"] += [e["down"][0].elapsed_time(e["down"][1]) for e in evs.values()]
        ms, n = _read_attn_timer()
        k["attn"][0] += ms
        k["attn"][1] += n
    return kinds


def _summarize(kinds, cfg, Tq, Tk):
    """Per step kind: mean step time, salient rows per layer, and the mean launch time and
    algorithmic work of the fused attention kernel and of the two FFN GEMMs."""
    hid, inter = cfg["hidden"], cfg["inter"]
    L = cfg["prompt"] + cfg["response"]
    HD = cfg["heads"] * cfg["head_dim"]
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")
    per = {}
    for refresh, k in kinds.items():
        if not k["ms"]:
            continue
        n = mean(k["n_sal"])
        T = Tk if refresh else Tq
        attn_ms = k["attn"][0] / max(k["attn"][1], 1)
        af = _attn_flops(T, L, HD, n, n / cfg["batch"])
        per[refresh] = dict(ms=mean(k["ms"]), n=n, attn_ms=attn_ms, attn_flops=af,
                            attn_tf=af / (attn_ms * 1e-3) / 1e12, gate_ms=mean(k["gate"]),
                            down_ms=mean(k["down"]), gu_flops=2.0 * n * hid * 2 * inter, dn_flops=2.0 * n * inter * hid)
    return per


def time_config(name, cfg, steps, period, note):
    """Another configuration's sparse denoise steps (all its layers, the same timed step as
    config 1's), reported beside the config-1 line: step time at its cadence, tokens/s, and the
    fused attention and gate_up launches."""
    import torch

    layers = cfg["layers"]
    wl = build_workload(cfg, layers, "cuda:0", seed=1)
    wl["restore"]()
    wl["step"](refresh=False)
    torch.cuda.synchronize()
    kinds = _run_cadence(wl, steps, period, layers)
    Tq, Tk = wl["Tq"], wl["Tk"]
    per = _summarize(kinds, cfg, Tq, Tk)
    del wl
    torch.cuda.empty_cache()
    ms = (sum(kinds[False]["ms"]) + sum(kinds[True]["ms"])) / steps
    out = {"workload": f"{name}: {note}", "layers": layers, "batch": cfg["batch"],
           "seq_len": cfg["prompt"] + cfg["response"], "response_len": cfg["response"], "hidden": cfg["hidden"],
           "heads": cfg["heads"], "kv_heads": cfg["kv_heads"], "ffn": cfg["inter"], "tau": cfg["tau"],
           "perturbed": cfg["perturb"], "steps": steps, "refresh_every": period,
           "ms_per_step": round(ms, 4), "tokens_per_s": round(Tq / (ms / 1e3), 1)}
    for refresh, key in ((False, "q_pruned"), (True, "refresh")):
        if refresh not in per:
            continue
        r = per[refresh]
        out[key] = {"ms_per_step": round(r["ms"], 4), "avg_salient_rows_per_layer": round(r["n"], 1),
                    "attention_us": round(r["attn_ms"] * 1e3, 2),
                    "attention_tflops": round(r["attn_tf"], 1),
                    "attention_frac": round(r["attn_tf"] / PEAK_BF16_TFLOPS, 4),
                    "gate_up_us": round(r["gate_ms"] * 1e3, 2),
                    "gate_up_frac": round(r["gu_flops"] / (r["gate_ms"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                    "down_us": round(r["down_ms"] * 1e3, 2)}
    print(f"[bench] {name}: {ms:.3f} ms/step, {out['tokens_per_s']:.0f} tokens/s", file=sys.stderr, flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=8, help="timed denoise steps; step i is a refresh step when "
                                                            "i %% 4 == 3 (config 1's cadence)")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=None, help="debug only: fewer layers than the model has")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true", help="skip the config-2 / config-4 step lines")
    ap.add_argument("--profile-gate-up", action="store_true",
                    help="run only the gate_up GEMM + a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--profile-attention", action="store_true",
                    help="run only the standalone row-sparse and column-sparse attention tiles (for rocprofv3 --pmc)")
    ap.add_argument("--perturb", type=float, default=None,
                    help="config 1's perturbed fraction of the response rows (default 0.15); the PMC traffic "
                         "figures apply to the default only")
    ap.add_argument("--probe-issue", action="store_true",
                    help="MFMA / VALU issue probe of one SIMD (dyllm_issue_probe): cycles per loop iteration of "
                         "each kind alone and both in one wavefront; prints one JSON line")
    ap.add_argument("--profile-hbm", action="store_true",
                    help="run only the standalone HBM-bound kernels at the config-1 shape and print their GB/s")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU; the hot path is not sharded across GPUs "
              "(sequences would split across data-parallel ranks with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from dyllm_amd import _lib

    cfg = dict(CONFIG1)
    if args.perturb is not None:
        if not 0.0 < args.perturb < 1.0:
            print("bench.py: --perturb must lie in (0, 1)", file=sys.stderr)
            sys.exit(2)
        cfg["perturb"] = args.perturb
    default_mix = cfg["perturb"] == CONFIG1["perturb"]
    if args.profile_gate_up:
        profile_gate_up(cfg)
        return
    if args.profile_hbm:
        profile_hbm(cfg)
        return
    if args.profile_attention:
        profile_attention(cfg)
        return
    if args.probe_issue:
        probe_issue()
        return
    layers = args.layers or cfg["layers"]
    dev = "cuda:0"
    torch.cuda.set_device(0)
    print(f"[bench] building config-1 workload ({layers} layers)", file=sys.stderr, flush=True)
    wl = build_workload(cfg, layers, dev)
    for i in range(args.warmup):
        wl["restore"]()
        wl["step"](refresh=(i % 2 == 1))
    torch.cuda.synchronize()

    kinds = _run_cadence(wl, args.steps, 4, layers)
    total_ms = sum(kinds[False]["ms"]) + sum(kinds[True]["ms"])
    ms_per_step = total_ms / args.steps
    # the same cadence with the salient-row K/V projection GEMM added per layer (the model's step
    # includes it; `value` covers the path of the saliency layer, attention through FFN)
    wl["restore"]()
    wl["step"](refresh=False, with_kv_proj=True)
    torch.cuda.synchronize()
    kinds_kv = _run_cadence(wl, args.steps, 4, layers, with_kv_proj=True)
    ms_kv = (sum(kinds_kv[False]["ms"]) + sum(kinds_kv[True]["ms"])) / args.steps
    Tq, Tk = wl["Tq"], wl["Tk"]
    value = Tq / (ms_per_step / 1e3)     # B x Lq denoised tokens per step, at the config-1 cadence

    hid, inter = cfg["hidden"], cfg["inter"]
    L = cfg["prompt"] + cfg["response"]
    per = _summarize(kinds, cfg, Tq, Tk)
    q = per[False]
    print(f"[bench] {ms_per_step:.3f} ms/step at the cadence; Q-pruned {q['ms']:.3f} ms "
          f"({q['n']:.0f} salient rows/layer), attention {q['attn_ms'] * 1e3:.1f} us -> {q['attn_tf']:.1f} TFLOP/s, "
          f"gate_up {q['gate_ms'] * 1e3:.1f} us, down {q['down_ms'] * 1e3:.1f} us", file=sys.stderr, flush=True)
    if True in per:
        r = per[True]
        print(f"[bench] refresh {r['ms']:.3f} ms, attention {r['attn_ms'] * 1e3:.1f} us -> {r['attn_tf']:.1f} TFLOP/s",
              file=sys.stderr, flush=True)
    avg_n = q["n"]
    gate_bm = _lib.load().dyllm_ffn_tile_rows(int(round(avg_n)), 2 * inter, hid, 1)
    down_bm = _lib.load().dyllm_ffn_tile_rows(int(round(avg_n)), hid, inter, 0)

    def rf(kernel, flops, ms, traffic=None, algo_bytes=None, note=None):
        tf = flops / (ms * 1e-3) / 1e12
        d = {"kernel": kernel, "bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
             "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
             "avg_launch_us": round(ms * 1e3, 2), "flop_per_launch": flops}
        if traffic is not None:
            d["traffic_unit"] = "bytes per launch (PMC)"
        if algo_bytes is not None:
            d["algorithmic_bytes"] = algo_bytes
        if note:
            d["note"] = note
        return d

    rf_attn = rf("attention_step_kernel<4> (fused Q-pruned step: row-sparse + column-sparse tiles)",
                 q["attn_flops"], q["attn_ms"], ATTN_TRAFFIC_BYTES if default_mix else None,
                 345.0e6 if default_mix else None,
                 "bound by its VALU plus MFMA issue (softmax over all query-key pairs); frac counts algorithmic "
                 "MFMA work only")
    rf_gate = rf(f"gemm_kernel<{gate_bm},4,SwiGLU> (gathered gate_up + SiLU*up, tile {gate_bm}x256)",
                 q["gu_flops"], q["gate_ms"], GATE_UP_TRAFFIC_BYTES if default_mix else None,
                 231.4e6 if default_mix else None)
    rf_down = rf(f"gemm_kernel<{down_bm},4,Store> down + FFN-cache scatter (+ split-K reduction)",
                 q["dn_flops"], q["down_ms"])
    # the dominant kernel (longest mean launch) carries "roofline", the other one rides along
    if q["attn_ms"] >= q["gate_ms"]:
        rf_main, rf_other_key, rf_other = rf_attn, "roofline_gate_up", rf_gate
    else:
        rf_main, rf_other_key, rf_other = rf_gate, "roofline_attention", rf_attn
    extra = {}
    if True in per:
        r = per[True]
        extra["refresh_step"] = {"ms_per_step": round(r["ms"], 4), "tokens_per_s": round(Tq / (r["ms"] / 1e3), 1),
                                 "queried_rows": Tk, "avg_salient_rows_per_layer": round(r["n"], 1),
                                 "roofline_attention": rf("attention_step_kernel<4> (fused refresh step, every row "
                                                          "queried)", r["attn_flops"], r["attn_ms"])}
    extra["q_pruned_step"] = {"ms_per_step": round(q["ms"], 4), "tokens_per_s": round(Tq / (q["ms"] / 1e3), 1)}
    extra["step_with_kv_projection"] = {
        "ms_per_step": round(ms_kv, 4), "tokens_per_s": round(Tq / (ms_kv / 1e3), 1),
        "note": "the same cadence with the salient-row K/V projection GEMM (dyllm_linear) added per layer, "
                "as the model's sparse step runs it; its output is not consumed (the K/V epilogue keeps "
                "the stand-in rows, so the salient fraction stays as built)"}
    print(f"[bench] with the K/V projection: {ms_kv:.3f} ms/step, {Tq / (ms_kv / 1e3):.0f} tokens/s",
          file=sys.stderr, flush=True)
    del wl
    torch.cuda.empty_cache()
    extra["roofline_down"] = rf_down
    extra["roofline_dense_attention"] = time_dense_attention(cfg)
    extra["roofline_moe_config3"] = time_moe()
    kv_proj = time_kv_projection(cfg, int(round(avg_n)))
    print(f"[bench] dense attention {extra['roofline_dense_attention']['avg_launch_us']:.1f} us, "
          f"MoE (config 3) {extra['roofline_moe_config3']['avg_launch_us']:.1f} us -> "
          f"{extra['roofline_moe_config3']['achieved']:.1f} TFLOP/s, kv projection {kv_proj['avg_launch_us']:.1f} us",
          file=sys.stderr, flush=True)

    if not args.no_other_configs:
        extra["config2_step"] = time_config("config2", CONFIG2, 4, 4, "Dream-v0-7B shape (GQA 28/4, FFN 18944), "
                                            "B=16 x (512+1536), 25 % perturbed, refresh every 4th step")
        extra["config4_step"] = time_config("config4", CONFIG4, 8, 8, "LLaDA-8B shape, B=2 x (2048+6144), "
                                            "tau 0.995, 5 % perturbed, refresh every 8th step")

    cpu = None
    if not args.no_cpu_baseline:
        # the box allots 16 host threads to a one-GPU job (OMP_NUM_THREADS); os.cpu_count() counts
        # the whole host, whose cores other jobs share
        threads = min(int(os.environ.get("OMP_NUM_THREADS", "16") or 16), os.cpu_count() or 1)
        print(f"[bench] CPU baseline on {threads} threads (host reports {os.cpu_count()} CPUs)",
              file=sys.stderr, flush=True)
        cpu = cpu_baseline(cfg, int(round(avg_n)), threads)

    line = {
        "metric": "salient-path tokens/s per denoise step, LLaDA-8B shape bf16; % HBM/MFMA roofline",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic (random-init N(0,0.02) weights, N(0,1) K/V/Q, {cfg['perturb'] * 100:g}% perturbed "
                "response rows)",
        "config": {"workload": "config1: LLaDA-8B shape, sparse denoise steps over 32 layers at the config-1 "
                               "cadence (3 Q-pruned : 1 refresh)",
                   "layers": layers, "batch": cfg["batch"], "seq_len": L, "response_len": cfg["response"],
                   "hidden": hid, "heads": cfg["heads"], "ffn": inter, "tau": cfg["tau"],
                   "perturbed": cfg["perturb"], "q_pruned_steps": len(kinds[False]["ms"]), "refresh_steps": len(kinds[True]["ms"]),
                   "avg_salient_rows_per_layer": round(avg_n, 1)},
        "roofline": rf_main,
        rf_other_key: rf_other,
        **extra,
        "cpu_baseline": cpu,
        "kv_projection": kv_proj,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
