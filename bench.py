"""Benchmark of the quantize-and-score hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]

Headline: 4-bit packed-code inner-product top-k scan over
N = 10,000,000 L2-normalized N(0,1) vectors, d = 128, one fp16 normalized query per
step, k = 10.  A step is one `ip_scan_topk_pairs` call -- the scan TurboQuantIndex runs
on its 4-bit database, held in the pair layout (the same 64 bytes per row as the
bit-plane rows, rearranged) -- query rotation + table build, the ADC scan, the top-k
merge, with the database resident in HBM.  `value` is queries/s.  The same scan over
the reference's bit-plane rows is reported beside it under "extra".

Also measured in the same run and reported under "extra": the Q = 64 / 1024 batches
and the 3- and 2-bit databases of the same config; fused GQA decode attention over a
packed KV cache (configs[3]: B=32, Hq=32, Hkv=8, d=64, K4/V2, T = 4K/16K/32K);
quantize throughput (configs[2]: prod 3+1 bit, N=1M d=128 and N=390k d=200); prod-mode
index search over 10M x 128 rows of 3-bit codes + QJL signs.

roofline: the scan op's algorithmic bytes (N*(b*16 + 4) + Q*d*2 + Q*k*12) over its
average duration from HIP events on the launch stream; peak = 8 TB/s.
cpu_baseline: the reference's own C++ core (search_packed, compiled from the
reference's sources into oracle/_ref) -- or this repo's C port of it when that build
is absent -- timed on this host's cores on a bounded sample of the same database.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "turboquant-kv_amd"))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 (vector or MFMA)
METRIC = "packed-KV decode-attn GB/s (% HBM peak); 10M×d128 4-bit IP scan queries/s"
PUBLISHED_QPS = 1000.0 / 2.70  # the reference's published H100 Triton scan: 1 query, 2.70 ms
# HBM bytes per launch of pair_filter_kernel<128,false> on the headline workload, from
# rocprofv3 FETCH_SIZE + WRITE_SIZE passes scaled by a copy kernel's readings (FETCH x2.0,
# WRITE x1.0); commands and raw counts in profiles/pair_filter_kernel_b4_q1_N10M_d128.md.
SCAN_TRAFFIC_BYTES = 681.0e6


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_op(fn, steps, warmup, settle_s=0.0):
    """Mean ms per call of `steps` calls after `warmup` untimed ones.  settle_s: before
    the warm-up, keep calling fn for that long (untimed), so the GPU's clocks have settled
    under this kernel's sustained load (a fresh box runs the first ~100 ms of a kernel up
    to 20 % slower)."""
    import torch

    if settle_s > 0:
        t_end = time.perf_counter() + settle_s
        while time.perf_counter() < t_end:
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms


def make_db(n, d, bits, seed=0):
    import torch
    from turboquant_kv import _lib
    from turboquant_kv.codebook import lloyd_max_codebook, make_rotation_matrix

    ops = _lib.ops()
    g = torch.Generator(device="cuda").manual_seed(seed)
    R = make_rotation_matrix(d, 42).cuda()
    bnd, cen = lloyd_max_codebook(bits, d)
    packed = torch.empty(n, bits * ((d + 7) // 8), dtype=torch.uint8, device="cuda")
    norms = torch.empty(n, dtype=torch.float32, device="cuda")
    chunk = 2_000_000
    qt = 0.0
    for c in range(0, n, chunk):
        m = min(chunk, n - c)
        x = torch.randn(m, d, generator=g, device="cuda")
        x = x / x.norm(dim=1, keepdim=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        p, nm = ops.quantize_mse_packed(x, R, bnd.cuda(), bits)
        torch.cuda.synchronize()
        qt += time.perf_counter() - t0
        packed[c:c + m] = p
        norms[c:c + m] = nm
        del x, p, nm
    return packed, norms, R, cen.cuda(), qt


def queries(nq, d, seed=1):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(nq, d, generator=g, device="cuda")
    return (q / q.norm(dim=1, keepdim=True)).half()


def bench_scan(args, extra):
    import torch
    from turboquant_kv import _lib

    ops = _lib.ops()
    N, d, k = 10_000_000, 128, 10
    res = {}
    log("building the 10M x 128 4-bit database")
    packed, norms, R, cen, qt = make_db(N, d, 4)
    extra["quantize_mse_4bit_10M_d128"] = {"vectors_per_s": N / qt, "seconds": qt,
                                           "note": "fp32 input, host-timed, includes launch"}
    # TurboQuantIndex keeps 4-bit d=128 rows in the pair layout: same 64 bytes per row.
    pairs = torch.empty(1, N, d // 2, dtype=torch.uint8, device="cuda")
    ops.pack_decode_layout(packed.unsqueeze(0), pairs, d, 4, 0, 0)
    pairs = pairs[0]
    q1 = queries(1, d)
    bytes_alg = N * (4 * 16 + 4) + 1 * d * 2 + k * 12
    # The bit-plane comparison runs first: the GPU's clocks take a few milliseconds of
    # sustained load to settle, and the headline is timed after that.
    t = time_op(lambda: ops.ip_scan_topk(q1, packed, norms, cen, R, 4, k), 40, 3)
    extra["scan_b4_Q1_bitplane"] = {"us_per_query": t * 1e3, "queries_per_s": 1e3 / t,
                                    "GBps": bytes_alg / t / 1e6,
                                    "hbm_frac": bytes_alg / t / 1e6 / HBM_PEAK_GBS,
                                    "note": "same scan over the reference's bit-plane rows"}
    log(f"scan b=4 Q=1 (bit-plane rows): {t * 1e3:.1f} us/query, {bytes_alg / t / 1e6:.0f} GB/s")
    fn = lambda: ops.ip_scan_topk_pairs(q1, pairs, norms, cen, R, k)
    if not getattr(args, "batch_only", False):
        ms = time_op(fn, args.steps, args.warmup, settle_s=0.3)
        res["headline"] = (ms, bytes_alg)
        log(f"scan b=4 Q=1 (pair layout): {ms * 1e3:.1f} us/query, {bytes_alg / ms / 1e6:.0f} GB/s")
    if not args.quick:
        for Q, steps in ((64, 20), (1024, 5)):
            qq = queries(Q, d, seed=2)
            t = time_op(lambda: ops.ip_scan_topk_pairs(qq, pairs, norms, cen, R, k), steps, 2,
                        settle_s=0.1)
            # the multi-query filtered scan: one pass over the rows per 64-query tile, 2 d
            # flops per (query, row) of fp16 MFMA work in its filter
            tiles = (Q + 63) // 64
            flop = tiles * 64 * N * d * 2.0
            extra[f"scan_b4_Q{Q}"] = {
                "ms_per_batch": t, "queries_per_s": Q / t * 1e3,
                "row_passes": tiles, "GBps_rows_read": tiles * N * (4 * 16 + 4) / t / 1e6,
                "filter_TFLOPs": flop / t / 1e9, "fp16_dense_peak_frac": flop / t / 1e9 / 2500.0,
                "kernels": "mq_rotate + mq_tile + mq_sample + mq_filter + mq_merge (+ exact "
                           "scan for flagged queries: none here)"}
            log(f"scan b=4 Q={Q}: {t:.3f} ms/batch, {Q / t * 1e3:.0f} q/s, filter "
                f"{flop / t / 1e9:.0f} TFLOP/s, rows read at {tiles * N * 68 / t / 1e6:.0f} GB/s")
        # k = 100 (bench_realworld.py's recall@100 searches): the same fused kernels, one
        # query included (above k = 32 a single query takes the multi-query filter too)
        for Q, steps in ((1, 20), (64, 20), (1024, 5)):
            qq = queries(Q, d, seed=3)
            t = time_op(lambda: ops.ip_scan_topk_pairs(qq, pairs, norms, cen, R, 100), steps, 2,
                        settle_s=0.1)
            extra[f"scan_b4_Q{Q}_k100"] = {"ms_per_batch": t, "queries_per_s": Q / t * 1e3}
            log(f"scan b=4 Q={Q} k=100: {t:.3f} ms/batch, {Q / t * 1e3:.0f} q/s")
    # bit-plane rows (the CPU reference's input) and the pair rows the headline op reads
    res["db4"] = (packed, norms, R, cen, pairs)
    if not args.quick:
        for bits in (3, 2):
            # TurboQuantIndex keeps 2/3-bit d=128 rows as pair rows (same bytes per row)
            p3, n3, R3, c3, _ = make_db(N, d, bits)
            rows = ops.pack_pair_rows(p3, bits, d)
            ba = N * (bits * 16 + 4)
            if not getattr(args, "batch_only", False):
                # one query: the pair-row scan (one table read of two precomputed products
                # per pair of dims)
                t_bp = time_op(lambda: ops.ip_scan_topk(q1, p3, n3, c3, R3, bits, k), 20, 3)
                t = time_op(lambda: ops.ip_scan_topk_pair_rows(q1, rows, n3, c3, R3, bits, k), 30, 3)
                extra[f"scan_b{bits}_Q1"] = {"us_per_query": t * 1e3, "queries_per_s": 1e3 / t,
                                             "GBps": ba / t / 1e6, "hbm_frac": ba / t / 1e6 / HBM_PEAK_GBS,
                                             "layout": "pair rows (TurboQuantIndex storage)",
                                             "bitplane_rows_us": t_bp * 1e3}
                log(f"scan b={bits} Q=1: {t * 1e3:.1f} us, {ba / t / 1e6:.0f} GB/s "
                    f"(bit-plane rows {t_bp * 1e3:.1f} us)")
            for Q, steps in ((64, 20), (1024, 5)):
                # batches: the multi-query filtered scan over the pair rows (fp16 centroid
                # pairs from a 2^(2 bits)-entry table as the B operands)
                qq = queries(Q, d, seed=2)
                t = time_op(lambda: ops.ip_scan_topk_pair_rows(qq, rows, n3, c3, R3, bits, k), steps, 2,
                            settle_s=0.1)
                tiles = (Q + 63) // 64
                flop = tiles * 64 * N * d * 2.0
                extra[f"scan_b{bits}_Q{Q}"] = {
                    "ms_per_batch": t, "queries_per_s": Q / t * 1e3, "row_passes": tiles,
                    "GBps_rows_read": tiles * ba / t / 1e6, "filter_TFLOPs": flop / t / 1e9,
                    "fp16_dense_peak_frac": flop / t / 1e9 / 2500.0, "layout": "pair rows",
                    "kernels": "mq_rotate + mq_tile + mq_sample + mq_filter + mq_merge"}
                log(f"scan b={bits} Q={Q}: {t:.3f} ms/batch, {Q / t * 1e3:.0f} q/s, filter "
                    f"{flop / t / 1e9:.0f} TFLOP/s")
            del p3, n3, rows
    return res


def bench_decode(args, extra):
    import torch
    from turboquant_kv import _lib
    from turboquant_kv.codebook import lloyd_max_codebook, make_rotation_matrix

    ops = _lib.ops()
    B, Hq, Hkv, d, kb, vb = 32, 32, 8, 64, 4, 2
    Rk, Rv = make_rotation_matrix(d, 42).cuda(), make_rotation_matrix(d, 43).cuda()
    bk, ck = [t.cuda() for t in lloyd_max_codebook(kb, d)]
    bv, cv = [t.cuda() for t in lloyd_max_codebook(vb, d)]
    g = torch.Generator(device="cuda").manual_seed(0)
    out = {}
    for T in ((4096, 16384, 32768) if not args.quick else (32768,)):
        # rotate over enough caches to exceed the 256 MB Infinity Cache
        per = B * Hkv * T * (32 + 16 + 4 + 4)
        ncopies = max(1, math.ceil(1.2e9 / per)) if T < 32768 else 1
        caches = []
        for _ in range(ncopies):
            K = torch.randn(B, Hkv, T, d, generator=g, device="cuda").to(torch.bfloat16)
            V = torch.randn(B, Hkv, T, d, generator=g, device="cuda").to(torch.bfloat16)
            ch = torch.randint(0, d, (Hkv, 4), generator=g, device="cuda")
            for h in range(Hkv):
                K[:, h, :, ch[h]] *= 20
                V[:, h, :, ch[h]] *= 20
            kp, kn = ops.quantize_mse_packed(K.reshape(-1, d), Rk, bk, kb)
            vp, vn = ops.quantize_mse_packed(V.reshape(-1, d), Rv, bv, vb)
            del K, V
            # the decode layout QuantizedKVCache keeps (same bytes per token)
            kdl = torch.zeros(B * Hkv, T, d // 2, dtype=torch.uint8, device="cuda")
            vdl = torch.zeros(B * Hkv, T // 64, 16 * d, dtype=torch.uint8, device="cuda")
            ops.pack_decode_layout(kp.view(B * Hkv, T, -1), kdl, d, kb, 0, 0)
            ops.pack_decode_layout(vp.view(B * Hkv, T, -1), vdl, d, vb, 1, 0)
            caches.append((kp.view(B, Hkv, T, -1), kn.float().view(B, Hkv, T),
                           vp.view(B, Hkv, T, -1), vn.float().view(B, Hkv, T),
                           kdl.view(B, Hkv, T, -1), vdl.view(B, Hkv, T // 64, -1)))
            del kp, vp
        q = torch.randn(B, Hq, d, generator=g, device="cuda").to(torch.bfloat16)
        sl = torch.full((B,), T, dtype=torch.int32, device="cuda")
        it = [0]

        def fn():
            c = caches[it[0] % len(caches)]
            it[0] += 1
            return ops.decode_attention_dl(q, c[4], c[1], c[5], c[3], sl, ck, cv, Rk, Rv, 1.0 / 8.0)

        def fn_bitplane():
            c = caches[it[0] % len(caches)]
            it[0] += 1
            return ops.decode_attention_packed(q, c[0], c[1], c[2], c[3], sl, ck, cv, Rk, Rv, kb,
                                               vb, 1.0 / 8.0)

        # steady state: the first tens of calls of a kernel on a fresh box run slow (clocks,
        # first-touch of the cache copies); 200 calls of the short contexts take < 10 ms
        steps = 200 if T < 32768 else 40
        ms = time_op(fn, steps, 40, settle_s=0.3)
        ms_bp = time_op(fn_bitplane, steps, 40, settle_s=0.1)
        bytes_alg = per + 2 * B * Hq * d * 2
        out[T] = (ms, bytes_alg)
        extra[f"decode_attn_T{T}"] = {"us_per_step": ms * 1e3, "GBps": bytes_alg / ms / 1e6,
                                      "hbm_frac": bytes_alg / ms / 1e6 / HBM_PEAK_GBS,
                                      "tokens_per_s": B / ms * 1e3, "cache_copies": ncopies,
                                      "layout": "decode layout (QuantizedKVCache storage)",
                                      "bitplane_rows_us": ms_bp * 1e3,
                                      "bitplane_rows_GBps": bytes_alg / ms_bp / 1e6}
        log(f"decode T={T}: {ms * 1e3:.1f} us, {bytes_alg / ms / 1e6:.0f} GB/s "
            f"(bit-plane rows: {ms_bp * 1e3:.1f} us)")
        if T == 32768:
            # vLLM paging: the same rows in block pools of 16 tokens, blocks shuffled
            bs = 16
            nbs = T // bs
            perm = torch.randperm(B * nbs, generator=g, device="cuda")
            tab = perm.view(B, nbs).to(torch.int32)
            c = caches[0]

            def to_pool(x):  # [B, Hkv, T, ...] -> [B * nbs, Hkv, bs, ...] at the table's blocks
                y = x.reshape(B, Hkv, nbs, bs, *x.shape[3:]).transpose(1, 2)
                pool = torch.empty((B * nbs, Hkv, bs) + tuple(x.shape[3:]), dtype=x.dtype, device="cuda")
                pool[perm] = y.reshape(B * nbs, Hkv, bs, *x.shape[3:])
                return pool

            pk, pkn, pv, pvn = (to_pool(t) for t in c[:4])
            ms_pg = time_op(lambda: ops.decode_attention_paged(q, pk, pkn, pv, pvn, tab, sl, ck, cv,
                                                               Rk, Rv, kb, vb, 1.0 / 8.0), 20, 3, settle_s=0.1)
            extra[f"decode_attn_T{T}"].update({"paged_bs16_us": ms_pg * 1e3,
                                               "paged_bs16_GBps": bytes_alg / ms_pg / 1e6})
            log(f"decode T={T} paged (block 16, shuffled): {ms_pg * 1e3:.1f} us, "
                f"{bytes_alg / ms_pg / 1e6:.0f} GB/s")
            del pk, pv
            # the decode layout in the same block-16 pools (16-token value sub-blocks)
            pkp = to_pool(c[4])
            sub = c[5].reshape(B, Hkv, T // 64, 64, 4, 4).permute(0, 1, 2, 4, 3, 5)
            sub = sub.reshape(B, Hkv, nbs, 1, 4 * d).transpose(1, 2)
            pvs = torch.empty(B * nbs, Hkv, 1, 4 * d, dtype=torch.uint8, device="cuda")
            pvs[perm] = sub.reshape(B * nbs, Hkv, 1, 4 * d)
            ms_p16 = time_op(lambda: ops.decode_attention_paged_dl(q, pkp, pkn, pvs, pvn, tab, sl, ck,
                                                                   cv, Rk, Rv, 1.0 / 8.0), 20, 3, settle_s=0.1)
            extra[f"decode_attn_T{T}"].update({"paged_dl_bs16_us": ms_p16 * 1e3,
                                               "paged_dl_bs16_GBps": bytes_alg / ms_p16 / 1e6})
            log(f"decode T={T} paged decode layout (block 16, shuffled): {ms_p16 * 1e3:.1f} us, "
                f"{bytes_alg / ms_p16 / 1e6:.0f} GB/s")
            del pkp, pkn, pvs, pvn, sub
            # the decode layout in block pools of 64 tokens (one value tile per block),
            # blocks shuffled, read by the MFMA decode kernel through the table
            bs = 64
            nbs = T // bs
            perm = torch.randperm(B * nbs, generator=g, device="cuda")
            tab = perm.view(B, nbs).to(torch.int32)
            pkn, pvn = to_pool(c[1]), to_pool(c[3])
            pkp = to_pool(c[4])
            pvt = torch.empty(B * nbs, Hkv, 1, 16 * d, dtype=torch.uint8, device="cuda")
            pvt[perm] = c[5].transpose(1, 2).reshape(B * nbs, Hkv, 1, 16 * d)
            ms_pdl = time_op(lambda: ops.decode_attention_paged_dl(q, pkp, pkn, pvt, pvn, tab, sl, ck,
                                                                   cv, Rk, Rv, 1.0 / 8.0), 20, 3, settle_s=0.1)
            extra[f"decode_attn_T{T}"].update({"paged_dl_bs64_us": ms_pdl * 1e3,
                                               "paged_dl_bs64_GBps": bytes_alg / ms_pdl / 1e6})
            log(f"decode T={T} paged decode layout (block 64, shuffled): {ms_pdl * 1e3:.1f} us, "
                f"{bytes_alg / ms_pdl / 1e6:.0f} GB/s")
            del pkp, pkn, pvt, pvn
            # configs[4]'s K4/V3 cache in vLLM's default block-16 pools, blocks shuffled:
            # random codes and norms (the kernel's time does not depend on their values)
            bs, vb3 = 16, 3
            nbs = T // bs
            perm = torch.randperm(B * nbs, generator=g, device="cuda")
            tab = perm.view(B, nbs).to(torch.int32)
            pkp = torch.randint(0, 256, (B * nbs, Hkv, bs, d // 2), dtype=torch.uint8, device="cuda",
                                generator=g)
            pv3 = torch.randint(0, 256, (B * nbs, Hkv, bs // 16, 128 * vb3), dtype=torch.uint8,
                                device="cuda", generator=g)
            pkn = torch.rand(B * nbs, Hkv, bs, generator=g, device="cuda") + 0.5
            pvn = torch.rand(B * nbs, Hkv, bs, generator=g, device="cuda") + 0.5
            cv3 = lloyd_max_codebook(vb3, d)[1].cuda()
            ms_v3 = time_op(lambda: ops.decode_attention_paged_dl(q, pkp, pkn, pv3, pvn, tab, sl, ck,
                                                                  cv3, Rk, Rv, 1.0 / 8.0), 20, 3, settle_s=0.1)
            bytes_v3 = B * Hkv * T * (d // 2 + 8 * vb3 + 4 + 4) + 2 * B * Hq * d * 2
            extra["decode_attn_T32768_paged_K4V3_bs16"] = {
                "us_per_step": ms_v3 * 1e3, "GBps": bytes_v3 / ms_v3 / 1e6,
                "hbm_frac": bytes_v3 / ms_v3 / 1e6 / HBM_PEAK_GBS, "tokens_per_s": B / ms_v3 * 1e3,
                "layout": "decode-layout pools, block 16 (16-token value sub-blocks of 384 B)",
                "bytes_per_token_head": d // 2 + 8 * vb3 + 8}
            log(f"decode T={T} paged K4/V3 decode layout (block 16, shuffled): {ms_v3 * 1e3:.1f} us, "
                f"{bytes_v3 / ms_v3 / 1e6:.0f} GB/s")
            del pkp, pkn, pv3, pvn
            # head_dim 128 (the Llama-3-8B / Qwen-7B head shape), contiguous decode layout,
            # K4/V2 and K4/V3: random codes and norms (the kernel's time does not depend on them)
            d2 = 128
            Rk2 = make_rotation_matrix(d2, 42).cuda()
            Rv2 = make_rotation_matrix(d2, 43).cuda()
            ck2 = lloyd_max_codebook(4, d2)[1].cuda()
            q2 = torch.randn(B, Hq, d2, generator=g, device="cuda").to(torch.bfloat16)
            kp2 = torch.randint(0, 256, (B, Hkv, T, d2 // 2), dtype=torch.uint8, device="cuda", generator=g)
            kn2 = torch.rand(B, Hkv, T, generator=g, device="cuda") + 0.5
            vn2 = torch.rand(B, Hkv, T, generator=g, device="cuda") + 0.5
            for vbh in (2, 3):
                vt2 = torch.randint(0, 256, (B, Hkv, T // 64, 8 * vbh * d2), dtype=torch.uint8,
                                    device="cuda", generator=g)
                cv2 = lloyd_max_codebook(vbh, d2)[1].cuda()
                ms_h = time_op(lambda: ops.decode_attention_dl(q2, kp2, kn2, vt2, vn2, sl, ck2, cv2, Rk2,
                                                               Rv2, 1.0 / math.sqrt(d2)), 20, 3, settle_s=0.1)
                bytes_h = B * Hkv * T * (d2 // 2 + vbh * d2 // 8 + 8) + 2 * B * Hq * d2 * 2
                extra[f"decode_attn_T{T}_d128_K4V{vbh}"] = {
                    "us_per_step": ms_h * 1e3, "GBps": bytes_h / ms_h / 1e6,
                    "hbm_frac": bytes_h / ms_h / 1e6 / HBM_PEAK_GBS, "tokens_per_s": B / ms_h * 1e3,
                    "config": f"B {B}, Hq {Hq}, Hkv {Hkv}, head_dim 128, bf16 queries, fp32 norms"}
                log(f"decode T={T} head_dim 128 K4/V{vbh}: {ms_h * 1e3:.1f} us, "
                    f"{bytes_h / ms_h / 1e6:.0f} GB/s")
                del vt2
            del kp2, kn2, vn2
        del caches
    return out


def bench_prefill(args, extra):
    """Causal prefill of a 4096-token prompt over decode-layout paged pools (block 16, the
    vLLM default), Llama-3.2-1B attention shape (Hq 32, Hkv 8, d 64), K4/V2, one layer:
    the tiled prefill kernel against the per-token decode launch it replaces."""
    import torch
    from turboquant_kv import _lib
    from turboquant_kv.config import TurboQuantConfig
    from turboquant_kv.vllm_plugin import PagedKVPools

    ops = _lib.ops()
    Hq, Hkv, d, bs, n = 32, 8, 64, 16, 4096
    nb = n // bs + 8
    pools = PagedKVPools(TurboQuantConfig(), 1, nb, bs, Hkv, d, "cuda", layout="decode")
    g = torch.Generator(device="cuda").manual_seed(11)
    table = torch.randperm(nb, generator=g, device="cuda")[:n // bs].to(torch.int32)
    pos = torch.arange(n, device="cuda")
    slots = table.long()[pos // bs] * bs + pos % bs
    k = torch.randn(n, Hkv, d, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(n, Hkv, d, generator=g, device="cuda").to(torch.bfloat16)
    pools.write(0, k, v, slots)
    q = torch.randn(n, Hq, d, generator=g, device="cuda").to(torch.bfloat16)
    scale = 1.0 / 8.0
    ms = time_op(lambda: pools.prefill(0, q, table, n, scale), 20, 3, settle_s=0.1)
    st = pools.layers[0]
    bt = table[None].expand(n, -1).contiguous()
    lens = torch.arange(1, n + 1, dtype=torch.int32, device="cuda")
    ms_tok = time_op(lambda: ops.decode_attention_paged_dl(q, st["kp"], st["kn"], st["vt"], st["vn"], bt,
                                                           lens, pools.kcen, pools.vcen, pools.R_k,
                                                           pools.R_v, scale), 5, 1)
    flop = Hq * n * (n + 1) / 2 * 4 * d  # q.k and w.v over the visible (query, token) pairs
    extra["prefill_paged_dl_4096_llama1b"] = {
        "ms_per_layer": ms, "tokens_per_s": n / ms * 1e3, "TFLOPs": flop / ms / 1e9,
        "fp16_dense_peak_frac": flop / ms / 1e9 / 2500.0,
        "kernel": "dl_prefill_kernel<true,false> (block 16, bf16 queries)",
        "per_token_decode_ms": ms_tok,
        "note": "one layer, 4096 new tokens at positions 0..4095 (T = n), bf16 queries, fp32 out; "
                "TFLOP/s counts 4 d flop per visible (query head, token) pair; with bf16 queries "
                "the kernel runs one fp16 MFMA product per term (fp32/fp16 queries take hi/lo "
                "parts, 3 MFMAs per term) and three 16-row query groups per wave"}
    log(f"prefill 4096 tokens (paged decode layout, block 16): {ms:.3f} ms per layer, "
        f"{n / ms * 1e3 / 1e6:.2f} M tokens/s, {flop / ms / 1e9:.1f} TFLOP/s; per-token decode "
        f"launch {ms_tok:.3f} ms")


def bench_quantize(args, extra):
    import torch
    from turboquant_kv import _lib
    from turboquant_kv.codebook import lloyd_max_codebook, make_qjl_matrix, make_rotation_matrix

    ops = _lib.ops()
    g = torch.Generator(device="cuda").manual_seed(0)
    cases = [("prod_N1M_d128", 1_000_000, 128), ("prod_N390k_d200", 390_000, 200)]
    for name, n, d in cases:
        if d == 128:
            x = torch.clamp(torch.floor(torch.abs(torch.randn(n, d, generator=g, device="cuda") * 40)), 0, 255)
        else:
            sc = torch.exp(torch.randn(d, generator=g, device="cuda"))
            x = torch.randn(n, d, generator=g, device="cuda") * sc
        R = make_rotation_matrix(d, 42).cuda()
        S = make_qjl_matrix(d, d, 42).cuda()
        bnd, cen = [t.cuda() for t in lloyd_max_codebook(3, d)]
        ms = time_op(lambda: ops.quantize_prod_packed(x, R, bnd, cen, S, 4), 20, 5)
        bpp = (d + 7) // 8
        byts = n * (d * 4 + 3 * bpp + bpp + 8)
        flops = n * 6.0 * d * d  # three d x d contractions per vector
        tf = flops / ms / 1e9
        # fp32 MFMA kernels: d 128 with register-resident operands; d 200 padded to 208
        # with the operands reloaded per contraction (flops counted at the real d)
        kernel = ("quantize_mfma_kernel<true,128,7>" if d == 128
                  else "quantize_mfma_kernel<true,208,7,true>")
        extra[f"quantize_{name}"] = {
            "ms": ms, "vectors_per_s": n / ms * 1e3, "GBps": byts / ms / 1e6, "TFLOPs": tf,
            "roofline": {"bound": "mfma", "achieved": tf,
                         "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tf / FP32_PEAK_TFLOPS},
            "kernel": kernel}
        log(f"quantize {name}: {ms:.2f} ms, {n / ms * 1e3 / 1e6:.2f} M vec/s, {tf:.1f} TFLOP/s "
            f"({tf / FP32_PEAK_TFLOPS:.0%} of fp32 peak)")


def bench_formats(args, extra):
    """On-disk formats (host byte work): Huffman streams of 10M 4-bit code indices
    (HuffmanCoder encode / decode, native bit packing) and a TQIX v1 file of a 1M x 128
    4-bit index written and read back through TurboQuantIndex."""
    import os
    import tempfile
    import time

    import torch
    from turboquant_kv import EntropyPackedStorage, TurboQuantIndex

    g = torch.Generator().manual_seed(0)
    n = 10_000_000
    # codes distributed as the Lloyd-Max cells of N(0, 1) (what a quantizer emits)
    x = torch.randn(n, generator=g)
    edges = torch.tensor([-2.401, -1.844, -1.437, -1.099, -0.7996, -0.5224, -0.2582, 0.0,
                          0.2582, 0.5224, 0.7996, 1.099, 1.437, 1.844, 2.401])
    codes = torch.bucketize(x, edges).to(torch.uint8).view(-1, 128)
    t0 = time.perf_counter()
    st = EntropyPackedStorage.from_codes(codes, 4, 128)
    t1 = time.perf_counter()
    back = st.to_codes()
    t2 = time.perf_counter()
    assert torch.equal(back, codes)
    extra["huffman_4bit_10M"] = {"encode_Msym_per_s": n / (t1 - t0) / 1e6,
                                 "decode_Msym_per_s": n / (t2 - t1) / 1e6,
                                 "savings_pct": st.savings_pct, "threads": 1}
    log(f"huffman 10M 4-bit codes: encode {n / (t1 - t0) / 1e6:.0f} M sym/s, decode "
        f"{n / (t2 - t1) / 1e6:.0f} M sym/s, {st.savings_pct:.1f} % smaller")
    N, d = 1_000_000, 128
    idx = TurboQuantIndex(dim=d, bit_width=4, rotation="core", seed=7)
    idx.add(torch.randn(N, d, generator=g).cuda())
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "bench.tqix")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        idx.save_tqix(path)
        t1 = time.perf_counter()
        idx2 = TurboQuantIndex.load_tqix(path)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        size = os.path.getsize(path)
    assert idx2._norms.numel() == N
    extra["tqix_1M_d128_b4"] = {"bytes": size, "write_GBps": size / (t1 - t0) / 1e9,
                                "read_GBps": size / (t2 - t1) / 1e9,
                                "note": "host file I/O + device transfer, tmpfs or disk of the box"}
    log(f"TQIX 1M x 128 4-bit ({size / 1e6:.0f} MB): write {size / (t1 - t0) / 1e9:.2f} GB/s, "
        f"read {size / (t2 - t1) / 1e9:.2f} GB/s")


def bench_prod_scan(args, extra):
    """Prod-mode index search (TurboQuantIndex mode="prod", bit_width 4 = 3-bit MSE codes +
    1-bit QJL signs) over the headline's 10M x 128 shape: ip_scan_topk_prod scores the
    packed rows (72 B each); the reference's algorithm (search.py:229-252: dequantize_prod
    of every row, then q @ recon^T and topk) is timed beside it."""
    import torch
    from turboquant_kv import _lib
    from turboquant_kv.codebook import lloyd_max_codebook, make_qjl_matrix, make_rotation_matrix

    ops = _lib.ops()
    N, d, k, b = 10_000_000, 128, 10, 4
    g = torch.Generator(device="cuda").manual_seed(5)
    R = make_rotation_matrix(d, 42).cuda()
    S = make_qjl_matrix(d, d, 42).cuda()
    bnd, cen = [t.cuda() for t in lloyd_max_codebook(b - 1, d)]
    bpp = d // 8
    mp = torch.empty(N, (b - 1) * bpp, dtype=torch.uint8, device="cuda")
    sg = torch.empty(N, bpp, dtype=torch.uint8, device="cuda")
    rn = torch.empty(N, dtype=torch.float32, device="cuda")
    nm = torch.empty(N, dtype=torch.float32, device="cuda")
    chunk = 2_000_000
    for c in range(0, N, chunk):
        m = min(chunk, N - c)
        x = torch.randn(m, d, generator=g, device="cuda")
        x = x / x.norm(dim=1, keepdim=True)
        a, s_, r_, n_ = ops.quantize_prod_packed(x, R, bnd, cen, S, b)
        mp[c:c + m], sg[c:c + m], rn[c:c + m], nm[c:c + m] = a, s_, r_, n_
        del x, a, s_, r_, n_
    q1 = queries(1, d, seed=4)
    bytes_alg = N * ((b - 1) * bpp + bpp + 8) + d * 2 + k * 12
    # bit-plane MSE halves first (the comparison line), then the pair rows TurboQuantIndex
    # stores (same bytes per row, scores bit-identical)
    ms_bp = time_op(lambda: ops.ip_scan_topk_prod(q1, mp, sg, rn, nm, cen, R, S, b, k), 30, 3,
                    settle_s=0.1)
    rows = ops.pack_pair_rows(mp, b - 1, d)
    ms = time_op(lambda: ops.ip_scan_topk_prod_pair_rows(q1, rows, sg, rn, nm, cen, R, S, b, k), 30, 3,
                 settle_s=0.2)
    gbs = bytes_alg / ms / 1e6
    extra["scan_prod_b4_Q1"] = {
        "us_per_query": ms * 1e3, "queries_per_s": 1e3 / ms, "GBps": gbs,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "bytes_per_launch": bytes_alg},
        "kernel": "pair_scan_kernel<128,true,3,true> + merge_kernel (MSE half as pair rows)",
        "bitplane_rows_us": ms_bp * 1e3,
        "workload": "ip_scan_topk_prod N=10,000,000 d=128 bits=4 (3+1) Q=1 fp16 query k=10"}
    log(f"prod scan b=4 Q=1: {ms * 1e3:.1f} us/query, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.0%}); "
        f"bit-plane MSE rows {ms_bp * 1e3:.1f} us")
    del rows
    if not args.quick:
        qf = q1.float()

        def reference_algorithm():
            recon = ops.dequantize_prod_packed(mp, sg, rn, nm, cen, R, S, b, d)
            return torch.topk(qf @ recon.t(), k, dim=-1)

        t = time_op(reference_algorithm, 3, 1)
        extra["scan_prod_b4_Q1_dequantize_matmul"] = {
            "ms_per_query": t, "queries_per_s": 1e3 / t,
            "note": "the reference's prod search algorithm on this GPU (dequantize_prod kernel "
                    "+ torch matmul + topk), for comparison"}
        log(f"prod search by dequantize + matmul: {t:.2f} ms/query")


def bench_e2e(args, extra):
    """greedy decode through TurboQuantCache on a random-init Llama-3.2-1B-shaped
    model (16 layers, hidden 2048, 32 query / 8 KV heads of 64 dims, FFN 8192, vocab 128,256,
    tied embeddings, bf16): batch 64, 4096-token random-id prompts, 256 generated tokens,
    keys 4-bit / values 3-bit, fused attention (the decode kernel over the packed history,
    the exact new token merged by log-sum-exp).  Reports decode and end-to-end tokens/s,
    the decode kernel's time per layer at the final length with its HBM fraction, and the
    cache bytes against a bf16 cache of the same tokens; the same model with transformers'
    bf16 DynamicCache is timed beside it."""
    import torch
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM
    from turboquant_kv import TurboQuantCache, _lib
    from turboquant_kv.hf_integration import enable_fused_attention

    ops = _lib.ops()
    B, T0, n_new = 64, 4096, 256
    if args.quick:
        n_new = 64
    cfg = LlamaConfig(hidden_size=2048, intermediate_size=8192, num_hidden_layers=16,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=64,
                      vocab_size=128256, max_position_embeddings=8192, tie_word_embeddings=True,
                      rope_theta=500000.0)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    with torch.device("cuda"):
        model = LlamaForCausalLM(cfg).eval()
    torch.set_default_dtype(prev)
    g = torch.Generator(device="cuda").manual_seed(0)
    ids = torch.randint(0, cfg.vocab_size, (B, T0), generator=g, device="cuda")

    def run(cache):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.no_grad():
            out = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            toks = [nxt]
            for _ in range(n_new - 1):
                out = model(input_ids=nxt, past_key_values=cache, use_cache=True)
                nxt = out.logits[:, -1].argmax(-1, keepdim=True)
                toks.append(nxt)
            torch.cuda.synchronize()
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, torch.cat(toks, 1)

    cache = TurboQuantCache(key_bits=4, value_bits=3, fused_attention=True)
    enable_fused_attention(model)
    log("e2e: prefill + decode through TurboQuantCache K4/V3 (fused)")
    pre, dec, toks = run(cache)
    T = T0 + n_new - 1
    mem = cache.memory_bytes()
    bf16_bytes = cfg.num_hidden_layers * 2 * B * 8 * T * 64 * 2
    res = {"decode_tokens_per_s": B * (n_new - 1) / dec, "ms_per_decode_step": dec / (n_new - 1) * 1e3,
           "prefill_s": pre, "end_to_end_tokens_per_s": B * n_new / (pre + dec),
           "cache_bytes": mem, "cache_bytes_bf16": bf16_bytes, "compression_vs_bf16": bf16_bytes / mem,
           "batch": B, "prompt": T0, "new_tokens": n_new,
           "model": "random-init Llama-3.2-1B shape (16 x 2048, 32/8 heads x 64, FFN 8192, "
                    "vocab 128256, bf16)", "cache": "TurboQuantCache(key_bits=4, value_bits=3, "
                                                     "fused_attention=True)"}
    log(f"e2e K4/V3: prefill {pre:.2f} s, decode {dec / (n_new - 1) * 1e3:.2f} ms/step = "
        f"{B * (n_new - 1) / dec:.0f} tokens/s; cache {mem / 1e9:.2f} GB vs bf16 "
        f"{bf16_bytes / 1e9:.2f} GB ({bf16_bytes / mem:.2f}x)")
    # the decode kernel alone on the final caches, one call per layer in turn (16 x 146 MB:
    # beyond the 256 MB Infinity Cache)
    layers = cache.layers
    q = torch.randn(B, 32, 64, generator=g, device="cuda").to(torch.bfloat16)
    sl = torch.full((B,), T, dtype=torch.int32, device="cuda")
    it = [0]

    def one():
        L = layers[it[0] % len(layers)]
        it[0] += 1
        return ops.decode_attention_dl_lse(q, L.kp, L.kn, L.vp, L.vn, sl, L.kq.cen, L.vq.cen,
                                           L.kq.R, L.vq.R, 0.125)

    ms = time_op(one, 32, 4)
    nsz = layers[0].kn.element_size()  # bf16 norms in a bf16 model's cache (as the reference)
    kb = B * 8 * T * (32 + 24 + 2 * nsz) + 2 * B * 32 * 64 * 2
    res["decode_kernel_bytes_per_token_head"] = 32 + 24 + 2 * nsz
    res["decode_kernel_us_per_layer"] = ms * 1e3
    res["decode_kernel_GBps"] = kb / ms / 1e6
    res["decode_kernel_hbm_frac"] = kb / ms / 1e6 / HBM_PEAK_GBS
    log(f"e2e decode kernel (T={T}, K4/V3): {ms * 1e3:.1f} us per layer, {kb / ms / 1e6:.0f} GB/s")
    del cache, layers
    torch.cuda.empty_cache()
    if not args.quick:
        model.set_attn_implementation("sdpa")
        pre_b, dec_b, toks_b = run(DynamicCache())
        res["bf16_dynamic_cache"] = {"decode_tokens_per_s": B * (n_new - 1) / dec_b,
                                     "ms_per_decode_step": dec_b / (n_new - 1) * 1e3,
                                     "prefill_s": pre_b,
                                     "first_token_agreement": float((toks_b[:, 0] == toks[:, 0]).float().mean())}
        log(f"e2e bf16 DynamicCache: decode {dec_b / (n_new - 1) * 1e3:.2f} ms/step = "
            f"{B * (n_new - 1) / dec_b:.0f} tokens/s")
    extra["e2e_greedy_decode_llama1b_K4V3"] = res
    del model
    torch.cuda.empty_cache()


def bench_cpu_configs(args, extra):
    """CPU legs (the reference's CPU-runnable configurations) beside the GPU numbers of the same work:
    configs[0] in full -- TurboQuantMSE 4-bit on 65,536 N(0,1) fp32 vectors (torch CPU
    generator, seed 0), d = 128, R = make_rotation_matrix(128, 42), then 256 queries (the
    generator's next draws), k = 10 -- quantized by this repo's C/OpenMP restatement of
    csrc/cpu/quant_cpu.cpp:44-118 and searched by the reference's own core
    (turboquant_core.cpp:407-514, built into oracle/_ref; the C port where that build is
    absent); and configs[2]'s TurboQuantProd quantize (3-bit MSE + 1-bit QJL) on a
    bounded sample of its 1M x 128 heavy-tailed vectors through the numpy restatement of
    reference.py:392-469 (BLAS matmuls, the library's thread pool)."""
    import numpy as np
    import torch
    from turboquant_kv import _lib
    from turboquant_kv.codebook import lloyd_max_codebook, make_qjl_matrix, make_rotation_matrix

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cpu_libs
    import tq_oracle

    ops = _lib.ops()
    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    if not cpu_libs.have_port():
        log("cpu legs skipped: oracle/libtq_oracle_cpu.so is not built")
        return
    kind = "reference" if cpu_libs.have_ref() else "port"
    which = "ref" if cpu_libs.have_ref() else "port"
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(65536, 128, generator=gen)
    qs = torch.randn(256, 128, generator=gen)
    R = make_rotation_matrix(128, 42)
    bnd, cen = lloyd_max_codebook(4, 128)
    xn, Rn, bn, cn, qn = (t.numpy() for t in (x, R, bnd, cen, qs))
    # quantize: the reference's rotate_and_quantize_cpu (quant_cpu.cpp:44-118) compiled from
    # its source into oracle/_ref where that build exists, else the C restatement of it
    qref = cpu_libs.have_ref_cpu()
    quantize = cpu_libs.ref_cpu_rotate_and_quantize if qref else cpu_libs.rotate_and_quantize
    quantize(xn[:1024], Rn, bn, 4)  # warm the thread pool
    t0 = time.perf_counter()
    packed, norms = quantize(xn, Rn, bn, 4)
    tq = time.perf_counter() - t0
    t0 = time.perf_counter()
    s_cpu, i_cpu = cpu_libs.search_packed(qn, packed, norms, Rn, cn, 4, 10, which)
    ts = time.perf_counter() - t0
    # the same work on the GPU: quantize, then the 256-query scan over bit-plane rows
    xg, Rg, bg, cg, qg = (t.cuda() for t in (x, R, bnd, cen, qs))
    tgq = time_op(lambda: ops.quantize_mse_packed(xg, Rg, bg, 4), 20, 3)
    pg, ng = ops.quantize_mse_packed(xg, Rg, bg, 4)
    tgs = time_op(lambda: ops.ip_scan_topk(qg, pg, ng, cg, Rg, 4, 10), 20, 3)
    _, i_gpu = ops.ip_scan_topk(qg, pg, ng, cg, Rg, 4, 10)
    same = float((i_gpu.cpu().numpy() == i_cpu).mean())
    tqt, tst, pk_t, ids_t, thr = torch_cpu_config0(x, R, bnd, cen, qs)
    extra["cpu_config0_torch"] = {
        "quantize_vectors_per_s": 65536 / tqt, "search_queries_per_s": 256 / tst, "threads": thr,
        "kind": "port", "packed_byte_agreement_with_c_path": float((pk_t == packed).mean()),
        "topk_id_agreement_with_c_path": float((ids_t == i_cpu).mean()),
        "note": "torch-CPU composition of reference.py's algorithm: norm, divide, rotate, "
                "searchsorted, bit-plane pack; search by unpack, centroid gather, matmul, topk"}
    extra["cpu_config0"] = {
        "quantize_vectors_per_s": 65536 / tq, "search_queries_per_s": 256 / ts, "cores": cores,
        "quantize": ("reference (quant_cpu.cpp rotate_and_quantize_cpu, compiled from its source)"
                     if qref else "port (C/OpenMP restatement of quant_cpu.cpp:44-118)"),
        "search": f"{kind} (turboquant_core.cpp search_packed, one query per OpenMP thread)",
        "sample": "the whole config: 65,536 x 128 fp32 vectors, 256 queries, k = 10",
        "gpu_quantize_vectors_per_s": 65536 / tgq * 1e3, "gpu_search_queries_per_s": 256 / tgs * 1e3,
        "gpu_cpu_topk_id_agreement": same}
    log(f"config 0 CPU ({cores} threads): quantize {65536 / tq / 1e6:.2f} M vec/s, search "
        f"{256 / ts:.0f} q/s; GPU: {65536 / tgq * 1e3 / 1e6:.0f} M vec/s, {256 / tgs * 1e3:.0f} q/s")
    # configs[2] prod quantize on a bounded sample (100k of its 1M rows)
    n = 100_000
    xc = np.clip(np.floor(np.abs(rs_normal(n, 128) * 40)), 0, 255).astype(np.float32)
    S = make_qjl_matrix(128, 128, 42).numpy()
    b3, c3 = (t.numpy() for t in lloyd_max_codebook(3, 128))
    tq_oracle.quantize_prod(xc[:1000], 4, Rn, b3, c3, S)
    t0 = time.perf_counter()
    tq_oracle.quantize_prod(xc, 4, Rn, b3, c3, S)
    tp = time.perf_counter() - t0
    threads = cores
    try:
        from threadpoolctl import threadpool_info
        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=cores)
    except ImportError:
        pass
    extra["cpu_config2_quantize_prod"] = {
        "vectors_per_s": n / tp, "seconds": tp, "cores": threads, "kind": "port",
        "sample": f"{n} of config 2's 1M x 128 heavy-tailed fp32 vectors (floor(|N(0,40)|) "
                  "clipped to 255), prod 3+1 bit",
        "note": "numpy restatement of reference.py:392-469 (BLAS matmuls)"}
    log(f"config 2 prod quantize CPU ({threads} threads): {n / tp / 1e6:.2f} M vec/s")


def torch_cpu_config0(x, R, bnd, cen, qs, bits=4, k=10):
    """configs[0] through torch CPU ops in the steps of reference.py (quantize_mse:
    normalize by max(||x||, 1e-10), rotate, searchsorted, pack bit planes MSB first; search:
    unpack, centroids times norms, q_rot @ rows^T, topk).  Returns (quantize seconds,
    search seconds, packed codes, top-k ids, threads)."""
    import torch
    thr = torch.get_num_threads()
    n, d = x.shape
    w8 = torch.tensor([128, 64, 32, 16, 8, 4, 2, 1], dtype=torch.uint8)

    def quantize(v):
        nrm = torch.linalg.vector_norm(v, dim=1)
        u = v / nrm.clamp_min(1e-10)[:, None]
        codes = torch.searchsorted(bnd, (u @ R.T).contiguous())
        planes = [(((codes >> p) & 1).to(torch.uint8).view(v.shape[0], d // 8, 8) * w8).sum(-1, dtype=torch.uint8)
                  for p in range(bits)]
        return torch.cat(planes, dim=1), nrm

    def search(q, packed, nrm):
        planes = packed.view(-1, bits, d // 8)
        bitsv = ((planes[..., None] >> torch.arange(7, -1, -1, dtype=torch.uint8)) & 1).view(-1, bits, d)
        codes = (bitsv.to(torch.int64) << torch.arange(bits).view(1, bits, 1)).sum(1)
        rows = cen[codes] * nrm[:, None]
        return torch.topk((q @ R.T) @ rows.T, k, dim=1)

    quantize(x[:1024])
    t0 = time.perf_counter()
    packed, nrm = quantize(x)
    tq = time.perf_counter() - t0
    t0 = time.perf_counter()
    _, ids = search(qs, packed, nrm)
    ts = time.perf_counter() - t0
    return tq, ts, packed.numpy(), ids.numpy(), thr


def rs_normal(n, d, seed=0):
    import numpy as np
    return np.random.RandomState(seed).randn(n, d)


def cpu_baseline(db, budget_s=12.0):
    """The reference's C++ search_packed (turboquant_core.cpp:407-514, compiled from the
    reference's own source into oracle/_ref; "kind": "reference") -- or, where that build
    is absent, this repo's C restatement of it ("kind": "port") -- over the same 10M-row
    database, one query per OpenMP thread, enough rounds of queries for about `budget_s`
    seconds.  The same queries then run one at a time through the headline GPU op, and
    the fraction whose top-k ids and scores equal the CPU's bit for bit is reported: the
    full-size parity check of the timed path."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cpu_libs
    from turboquant_kv import _lib

    packed, norms, R, cen, pairs = db
    if not (cpu_libs.have_ref() or cpu_libs.have_port()):
        return None
    which = "ref" if cpu_libs.have_ref() else "port"
    kind = "reference" if which == "ref" else "port"
    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    p = packed.cpu().numpy()
    nm = norms.cpu().numpy()
    Rn, cn = R.cpu().numpy(), cen.cpu().numpy()
    qh = queries(cores * 64, 128, seed=3)
    qn = qh.float().cpu().numpy()
    t0 = time.perf_counter()
    cpu_libs.search_packed(qn[:cores], p, nm, Rn, cn, 4, 10, which)  # one query per thread
    t1 = time.perf_counter() - t0
    rounds = max(1, min(64, int(budget_s / max(t1, 1e-3))))
    nq = cores * rounds
    t0 = time.perf_counter()
    s_cpu, i_cpu = cpu_libs.search_packed(qn[:nq], p, nm, Rn, cn, 4, 10, which)
    dt = time.perf_counter() - t0
    ops = _lib.ops()
    same = 0
    for j in range(nq):
        s_g, i_g = ops.ip_scan_topk_pairs(qh[j:j + 1], pairs, norms, cen, R, 10)
        same += int(np.array_equal(i_g.cpu().numpy()[0], i_cpu[j])
                    and np.array_equal(s_g.cpu().numpy()[0].view(np.uint32),
                                       s_cpu[j].view(np.uint32)))
    log(f"cpu baseline ({kind}, {cores} threads): {nq / dt:.1f} q/s; GPU top-k bit-exact on "
        f"{same} of {nq} queries")
    name = ("turboquant_core.cpp search_packed compiled from the reference's source"
            if which == "ref" else "C restatement of turboquant_core.cpp search_packed")
    return {"value": nq / dt, "unit": "queries/s", "cores": cores, "kind": kind,
            "code": name,
            "sample": f"{nq} queries over all {p.shape[0]} rows of the same 4-bit database "
                      f"({dt:.1f} s, one query per OpenMP thread, k=10)",
            "cpu_gpu_topk_bit_exact": same / nq, "cpu_gpu_topk_queries_compared": nq}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline + T=32K decode only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quantize-only", action="store_true",
                    help="only the quantize_prod cases (configs 3a/3b), e.g. for a profiler run")
    ap.add_argument("--prod-only", action="store_true",
                    help="only the prod-mode scan (10M x 128, 3+1 bit), e.g. for a profiler run")
    ap.add_argument("--e2e-only", action="store_true",
                    help="only the end-to-end greedy decode (configs[4])")
    ap.add_argument("--scan-only", action="store_true",
                    help="only the index scans (configs[1]: 4-, 3- and 2-bit), e.g. for a profiler run")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode attention legs (configs[3] at 4K, 16K and 32K)")
    ap.add_argument("--batch-only", action="store_true",
                    help="only the 4-bit Q=64 / Q=1024 query batches of configs[1], e.g. for a profiler run")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 4096-token paged prefill, e.g. for a profiler run")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy 3 times (counter calibration)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": 1 << 30, "copy_bytes_written": 1 << 30, "launches": 3}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the path is single-GPU; there is no sharded run)", file=sys.stderr)
        sys.exit(2)
    import torch
    from turboquant_kv import _lib

    _lib.load()
    torch.cuda.init()
    if args.quantize_only:
        extra = {}
        bench_quantize(args, extra)
        print(json.dumps(extra))
        return
    if args.prod_only:
        extra = {}
        args.quick = True
        bench_prod_scan(args, extra)
        print(json.dumps(extra))
        return
    if args.e2e_only:
        extra = {}
        bench_e2e(args, extra)
        print(json.dumps(extra))
        return
    if args.decode_only:
        extra = {}
        dec = bench_decode(args, extra)
        extra["decode_attn_hbm_frac"] = {str(T): v[1] / v[0] / 1e6 / HBM_PEAK_GBS for T, v in dec.items()}
        print(json.dumps(extra))
        return
    if args.batch_only:
        extra = {}
        bench_scan(args, extra)
        print(json.dumps(extra))
        return
    if args.scan_only:
        extra = {}
        bench_scan(args, extra)
        print(json.dumps(extra))
        return
    if args.prefill_only:
        extra = {}
        bench_prefill(args, extra)
        print(json.dumps(extra))
        return
    extra = {}
    t0 = time.perf_counter()
    scan = bench_scan(args, extra)
    dec = bench_decode(args, extra)
    if not args.quick:
        bench_quantize(args, extra)
        bench_prod_scan(args, extra)
        bench_prefill(args, extra)
        bench_formats(args, extra)
        bench_e2e(args, extra)
    cpu = None if args.no_cpu else cpu_baseline(scan["db4"])
    if not args.no_cpu and not args.quick:
        bench_cpu_configs(args, extra)
    ms, bytes_alg = scan["headline"]
    achieved = bytes_alg / ms / 1e6
    value = 1e3 / ms
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": value / PUBLISHED_QPS,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "ip_scan_topk_pairs N=10,000,000 d=128 b=4 Q=1 (fp16 query) k=10",
                   "N": 10_000_000, "d": 128, "bits": 4, "queries_per_step": 1, "k": 10},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": SCAN_TRAFFIC_BYTES,
                     "kernel": "ip_scan_topk_pairs op (pair_filter_kernel<128,false> + filter_merge_kernel)",
                     "bytes_per_launch": bytes_alg},
        "cpu_baseline": cpu,
        "decode_attn_GBps": {str(T): v[1] / v[0] / 1e6 for T, v in dec.items()},
        "decode_attn_hbm_frac": {str(T): v[1] / v[0] / 1e6 / HBM_PEAK_GBS for T, v in dec.items()},
        "extra": extra,
        "wall_s": time.perf_counter() - t0,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
