"""Quantized-weight hot path on one MI355X: µs per layer, HBM GB/s, % of peak.

Headline (``value``): the 4-bit, group-64 quantized GEMV (M = 1) over a
[14336, 4096] weight with inputs resident in HBM and the weight buffers
rotated past the 256 MB Infinity Cache (cold), as achieved HBM GB/s of
algorithmic bytes.  One step is one decode token through a stack of 32 such
layers (each layer its own weight), so ``ms_per_step`` covers 32 GEMV calls
and ``config.us_per_layer`` is one call.  Timed with HIP events around a
HIP-graph replay of exactly ``--steps`` steps, so CPU launch cost is
excluded while every kernel of each call is included.

``detail`` holds the benchmark workloads: the dense [4096, 4096] GEMV and
the 4- and 8-bit [14336, 4096] / [4096, 14336] matmuls at M = 1, 16, 512
(cold and warm), the mx modes, KV append and quantized SDPA, packed VQ, then
the MoE experts (T = 1, 16, 256), the VQ experts (both codebooks, T = 1, 16)
and the KV8 decode (8k / 32k keys, L = 1 / 4; head dims 256 / 512).
``summary``, the line's last key, gives each workload's µs and % of its
bounding peak in one short string.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, published
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, published
CACHE_BYTES = 256 << 20        # Infinity Cache (MALL)
ROTATE_BYTES = 1 << 30         # rotate weight sets past this for cold numbers

METRIC = "quantized GEMV/MoE µs per layer + achieved HBM GB/s (% of peak) at M=1,16,512"


def _bound(nbytes, flops):
    """The roofline that bounds a call: MFMA when its FLOPs per byte exceed
    the ratio of the two published peaks (312.5), else HBM."""
    return "mfma" if flops / nbytes > (PEAK_BF16_TFLOPS * 1e12) / (PEAK_HBM_GBS * 1e9) else "hbm"


def dense_bytes(M, N, K, bits, gs=64):
    w = N * K * bits // 8 + 2 * 2 * N * (K // gs)      # packed + bf16 scales + biases
    return w + 2 * M * K + 2 * M * N


def make_sets(N, K, bits, cold, dev):
    import torch
    import knurlogic_amd as KA
    g = torch.Generator(device=dev).manual_seed(N * 7 + K + bits)
    w = (torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    base = KA.quantize(w, group_size=64, bits=bits)
    del w
    per = sum(t.numel() * t.element_size() for t in base)
    n = max(1, math.ceil(ROTATE_BYTES / per)) if cold else 1
    if cold:
        n = max(n, 4)
    sets = [base] + [tuple(t.clone() for t in base) for _ in range(n - 1)]
    return sets


def time_graph(fn_calls, replays=3, warm=1):
    """fn_calls(): enqueue the calls once.  Captured into one HIP graph,
    replayed `replays` times after `warm` untimed replays; returns mean ms
    per replay, timed with events on the capturing stream."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn_calls()                       # warm: allocator, code objects
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        fn_calls()
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        start.record(s)
        for _ in range(replays):
            graph.replay()
        end.record(s)
    end.synchronize()
    ms = start.elapsed_time(end) / replays
    del graph
    return ms


def bench_dense(bits, M, N, K, cold, calls, dev):
    import torch
    import knurlogic_amd as KA
    sets = make_sets(N, K, bits, cold, dev)
    g = torch.Generator(device=dev).manual_seed(M + N)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    ns = len(sets)

    def run():
        for i in range(calls):
            wq, s, b = sets[i % ns]
            KA.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits=bits)

    ms = time_graph(run) / calls
    us = ms * 1e3
    nbytes = dense_bytes(M, N, K, bits)
    flops = 2.0 * M * N * K
    gbs = nbytes / (us * 1e-6) / 1e9
    tfl = flops / (us * 1e-6) / 1e12
    bound = "mfma" if flops / nbytes > (PEAK_BF16_TFLOPS * 1e12) / (PEAK_HBM_GBS * 1e9) else "hbm"
    del sets
    torch.cuda.empty_cache()
    return {"op": "quantized_matmul", "bits": bits, "M": M, "N": N, "K": K,
            "cache": "cold" if cold else "warm", "us": round(us, 3),
            "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "TFLOPs": round(tfl, 2), "mfma_frac": round(tfl / PEAK_BF16_TFLOPS, 4),
            "bound": bound, "bytes": nbytes, "flops": flops}


def kv8_bytes(B, H, Hk, L, N, D, gs=64):
    kv = B * Hk * N * 2 * (D + (D // gs) * 2 * 2)       # K and V: bytes + bf16 scale/bias
    return kv + 2 * 2 * B * H * L * D                    # q in, out


def bench_kv8(B, H, Hk, L, N, D, cold, calls, dev):
    """8-bit-KV decode attention over quantized K/V caches of N keys, causal
    inside the L-token block; cold = K/V sets rotated past 1 GB."""
    import torch
    import knurlogic_amd as KA
    from knurlogic_amd import kvattn
    g = torch.Generator(device=dev).manual_seed(N + L)
    per = kv8_bytes(B, H, Hk, 0, N, D)
    n = max(4, math.ceil(ROTATE_BYTES / per)) if cold else 1
    sets = []
    for _ in range(n):
        trip = []
        for _kv in range(2):
            t = torch.randn(B * Hk * N, D, device=dev, generator=g).to(torch.bfloat16)
            wq, s, b = KA.quantize(t, group_size=64, bits=8)
            del t
            trip.append((wq.view(B, Hk, N, -1), s.view(B, Hk, N, -1), b.view(B, Hk, N, -1)))
        sets.append(tuple(trip))
    q = torch.randn(B, H, L, D, device=dev, generator=g).to(torch.bfloat16)
    mask = "causal" if L > 1 else None
    scale = D ** -0.5

    def run():
        for i in range(calls):
            K, V = sets[i % n]
            kvattn.decode_sdpa(q, K, V, scale, mask, 64, 8)

    us = time_graph(run) / calls * 1e3
    nbytes = kv8_bytes(B, H, Hk, L, N, D)
    flops = 4.0 * B * H * L * N * D
    gbs = nbytes / (us * 1e-6) / 1e9
    del sets
    torch.cuda.empty_cache()
    return {"op": "kv8_decode", "B": B, "H": H, "Hk": Hk, "L": L, "N": N, "D": D,
            "cache": "cold" if cold else "warm", "us": round(us, 3),
            "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "TFLOPs": round(flops / (us * 1e-6) / 1e12, 2),
            "mfma_frac": round(flops / (us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS, 4), "bound": _bound(nbytes, flops),
            "bytes": nbytes, "flops": flops}


def bench_qsdpa(B, H, Hk, L, N, D, bits, calls, dev):
    """mlx-lm's quantized attention (kvattn.quantized_sdpa: two
    kmi_qmm_batched products around kmi_masked_softmax) over quantized K/V
    of N keys, causal inside the L-token block; K/V sets rotated past 1 GB.
    Bytes: the packed K and V with their scales and biases, q in and out
    (the scores / probabilities round trip through L2 is not counted)."""
    import torch
    import knurlogic_amd as KA
    from knurlogic_amd import kvattn
    g = torch.Generator(device=dev).manual_seed(7000 + N + L)
    per = B * Hk * N * 2 * (D * bits // 8 + (D // 64) * 4)
    n = max(4, math.ceil(ROTATE_BYTES / per))
    sets = []
    for _ in range(n):
        trip = []
        for _kv in range(2):
            t = torch.randn(B * Hk * N, D, device=dev, generator=g).to(torch.bfloat16)
            wq, s, b = KA.quantize(t, group_size=64, bits=bits)
            del t
            trip.append((wq.view(B, Hk, N, -1), s.view(B, Hk, N, -1), b.view(B, Hk, N, -1)))
        sets.append(tuple(trip))
    q = torch.randn(B, H, L, D, device=dev, generator=g).to(torch.bfloat16)
    mask = "causal" if L > 1 else None
    scale = D ** -0.5

    def run():
        for i in range(calls):
            K, V = sets[i % n]
            kvattn.quantized_sdpa(q, K, V, scale, mask, 64, bits)

    us = time_graph(run) / calls * 1e3
    nbytes = per + 4 * B * H * L * D
    gbs = nbytes / (us * 1e-6) / 1e9
    del sets
    torch.cuda.empty_cache()
    return {"op": "quantized_sdpa", "B": B, "H": H, "Hk": Hk, "L": L, "N": N, "D": D, "bits": bits,
            "cache": "cold", "us": round(us, 3), "GBps": round(gbs, 1),
            "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm", "bytes": nbytes}


def bench_kv_append(B, Hk, S, D, bits, calls, dev):
    """Quantize-on-append into a quantized KV cache (kvcache.QuantKVCache's
    update_and_fetch): S new K and V rows of B x Hk heads quantized along D
    (group 64) straight into slab slots, K and V in one
    kmi_kv_quantize_append_kv launch; slots rotate through a 1 GB slab set
    so every write is cold.
    Bytes: K and V rows read (bf16) + packed words, scales and biases
    written."""
    import torch
    from knurlogic_amd import kvcache
    g = torch.Generator(device=dev).manual_seed(3000 + S)
    per_slot = B * Hk * (D * bits // 8 + (D // 64) * 4) * 2
    slots = max(S, (ROTATE_BYTES // per_slot) // S * S)
    k_parts = kvcache._alloc(B, Hk, slots, D, bits, 64, torch.bfloat16, dev)
    v_parts = kvcache._alloc(B, Hk, slots, D, bits, 64, torch.bfloat16, dev)
    xs = [torch.randn(B, Hk, S, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(2)]
    n_pos = slots // S

    def run():
        for i in range(calls):
            pos = (i % n_pos) * S
            kvcache.append_kv(k_parts, v_parts, xs[0], xs[1], pos, 64, bits)

    us = time_graph(run) / calls * 1e3
    nbytes = 2 * B * Hk * S * D * 2 + S * per_slot
    gbs = nbytes / (us * 1e-6) / 1e9
    del k_parts, v_parts
    torch.cuda.empty_cache()
    return {"op": "kv_append", "B": B, "Hk": Hk, "S": S, "D": D, "bits": bits, "cache": "cold",
            "us": round(us, 3), "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "bound": "hbm", "bytes": nbytes}


MOE = dict(E=128, k=8, H=2048, I=768, bits=4)


def moe_expert_bytes(H, I, bits, gs=64):
    per_matrix = H * I * bits // 8 + 2 * 2 * I * (H // gs)          # gate / up / down
    return 3 * per_matrix


def bench_moe(T, cold, calls, dev):
    """Qwen3.5-MoE-style experts: router (softmax, top-8, renormalize) from
    N(0, 1) logits, SwitchGLU over 4-bit g64 experts, weighted combine.
    Bytes: every routed expert's packed gate/up/down once + x and out."""
    import torch
    import knurlogic_amd as KA
    from knurlogic_amd import nn
    E, k, H, I, bits = MOE["E"], MOE["k"], MOE["H"], MOE["I"], MOE["bits"]
    g = torch.Generator(device=dev).manual_seed(1000 + T)
    per = E * moe_expert_bytes(H, I, bits)
    n = max(4, math.ceil(ROTATE_BYTES / per)) if cold else 1
    blocks = []
    for _ in range(n):
        w = [(torch.randn(*s, device=dev, generator=g) * 0.02).to(torch.bfloat16)
             for s in ((E, I, H), (E, I, H), (E, H, I))]
        blocks.append(nn.SparseMoeBlock(None, nn.SwitchGLU.from_float(*w, bits=bits), k))
        del w
    x = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, device=dev, generator=g).to(torch.bfloat16)
    inds, _ = KA.moe_route(logits, k)
    distinct = int(torch.unique(inds).numel())

    def run():
        for i in range(calls):
            blocks[i % n].experts(x, logits)

    us = time_graph(run) / calls * 1e3
    nbytes = distinct * moe_expert_bytes(H, I, bits) + 2 * 2 * T * H
    flops = 2.0 * T * k * 3 * H * I
    gbs = nbytes / (us * 1e-6) / 1e9
    del blocks
    torch.cuda.empty_cache()
    return {"op": "moe_experts", "T": T, "E": E, "top_k": k, "H": H, "I": I, "bits": bits,
            "experts_routed": distinct, "cache": "cold" if cold else "warm", "us": round(us, 3),
            "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "TFLOPs": round(flops / (us * 1e-6) / 1e12, 2),
            "mfma_frac": round(flops / (us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS, 4), "bound": _bound(nbytes, flops),
            "bytes": nbytes, "flops": flops}


def vq_expert_bytes(H, I, code_bytes):
    codes = (2 * I * (H // 8) + H * (I // 8)) * code_bytes          # gate, up, down indices
    return codes + 2 * (2 * I + H)                                   # fp16 per-channel scales


def bench_vq(T, kc, cold, calls, dev):
    """VQ experts at the Qwen3.5-MoE shape: 8-element vectors into a per-layer
    fp16 codebook (256 x 8 with uint8 indices, or 4096 x 8 with uint16),
    per-output-channel fp16 scales U(0.5, 1.5); router from N(0, 1) logits,
    fused gate/up + SwiGLU, down, weighted combine (one ``experts`` call:
    at one token the gate/up kernel routes it).  Bytes: every routed
    expert's indices and scales once, the codebook, x and out."""
    import torch
    import knurlogic_amd as KA
    from knurlogic_amd import nn
    E, k, H, I = MOE["E"], MOE["k"], MOE["H"], MOE["I"]
    cb_bytes = 1 if kc <= 256 else 2
    ct = torch.uint8 if cb_bytes == 1 else torch.uint16
    g = torch.Generator(device=dev).manual_seed(2000 + T + kc)
    per = E * vq_expert_bytes(H, I, cb_bytes)
    n = max(4, math.ceil(ROTATE_BYTES / per)) if cold else 1
    cb = (torch.randn(kc, 8, device=dev, generator=g) * 0.02).to(torch.float16)

    def mat(N, K):
        codes = torch.randint(0, kc, (E, N, K // 8), device=dev, generator=g, dtype=torch.int32).to(ct)
        sc = (torch.rand(E, N, device=dev, generator=g) + 0.5).to(torch.float16)
        return nn.VQSwitchLinear(codes, cb, sc)

    glus = [nn.VQSwitchGLU(mat(I, H), mat(I, H), mat(H, I)) for _ in range(n)]
    x = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, device=dev, generator=g).to(torch.bfloat16)
    inds, _ = KA.moe_route(logits, k)
    distinct = int(torch.unique(inds).numel())

    def run():
        for i in range(calls):
            glus[i % n].experts(x, logits, k)

    us = time_graph(run) / calls * 1e3
    nbytes = distinct * vq_expert_bytes(H, I, cb_bytes) + kc * 16 + 2 * 2 * T * H
    gbs = nbytes / (us * 1e-6) / 1e9
    del glus
    torch.cuda.empty_cache()
    return {"op": "vq_moe_experts", "T": T, "codebook": f"{kc}x8 fp16", "index_bytes": cb_bytes,
            "experts_routed": distinct, "cache": "cold" if cold else "warm", "us": round(us, 3),
            "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "TFLOPs": round(2.0 * T * k * 3 * H * I / (us * 1e-6) / 1e12, 2),
            "mfma_frac": round(2.0 * T * k * 3 * H * I / (us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "bound": _bound(nbytes, 2.0 * T * k * 3 * H * I), "bytes": nbytes, "flops": 2.0 * T * k * 3 * H * I}


def bench_vq_packed(T, calls, dev, dim=4, kc=2048, group=64, H=None, I=None):
    """VQ experts in the artifacts' packed layout, by default at the
    Qwen3.5-MoE shape: 11-bit fields (2048-entry codebook) of dim-4 vectors,
    per-group fp16 scales (64 inputs); router, gate/up + SwiGLU (one launch),
    down, weighted combine.  H / I / dim override the shape (the shipped
    Gemma-4 26B artifact: 128 experts, 2816 -> 704, dim-2 vectors).  Expert
    sets rotated past 1 GB.  Bytes: every routed expert's packed words and
    scales once, the codebook, x and out."""
    import torch
    import knurlogic_amd as KA
    from knurlogic_amd import nn
    E, k = MOE["E"], MOE["k"]
    H = MOE["H"] if H is None else H
    I = MOE["I"] if I is None else I
    bits = (kc - 1).bit_length()

    def mat_bytes(N, K):
        return N * ((K // dim + 31) // 32 * bits * 4 + K // group * 2)

    per_e = 2 * mat_bytes(I, H) + mat_bytes(H, I)
    n = max(4, math.ceil(ROTATE_BYTES / (E * per_e)))
    g = torch.Generator(device=dev).manual_seed(5000 + T)
    cb = (torch.randn(kc, dim, device=dev, generator=g) * 0.3).to(torch.float16)

    def mat(N, K):
        W = (K // dim + 31) // 32 * bits
        codes = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, N, W), device=dev, generator=g,
                              dtype=torch.int32).view(torch.uint32)
        sc = (torch.rand(E, N, K // group, device=dev, generator=g) + 0.5).to(torch.float16)
        return nn.VQSwitchLinear(codes, cb, sc, scale_group=group, pack_bits=bits, in_features=K)

    glus = [nn.VQSwitchGLU(mat(I, H), mat(I, H), mat(H, I)) for _ in range(n)]
    x = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, device=dev, generator=g).to(torch.bfloat16)
    inds, _ = KA.moe_route(logits, k)
    distinct = int(torch.unique(inds).numel())

    def run():
        for i in range(calls):
            glus[i % n].experts(x, logits, k)

    us = time_graph(run) / calls * 1e3
    nbytes = distinct * per_e + kc * dim * 2 + 2 * 2 * T * H
    gbs = nbytes / (us * 1e-6) / 1e9
    del glus
    torch.cuda.empty_cache()
    return {"op": "vq_packed_moe_experts", "T": T, "H": H, "I": I, "codebook": f"{kc}x{dim} fp16", "field_bits": bits,
            "experts_routed": distinct, "cache": "cold", "us": round(us, 3), "GBps": round(gbs, 1),
            "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm", "bytes": nbytes,
            "flops": 2.0 * T * k * 3 * H * I}


def bench_mx_moe(T, calls, dev, mode="mxfp4"):
    """MoE experts stored mxfp4 (E2M1 codes, E8M0 scales per 32 inputs, the
    routed-expert format of DeepSeek-V4 checkpoints) at the Qwen3.5-MoE
    shape through SwitchGLU: router, then gate/up + SwiGLU and down + the
    weighted combine (token-major kernels up to 16 pairs, else gather_qmm
    for the stacked gate|up, SwiGLU, down and the combine).  Expert sets
    rotated past 1 GB.  Bytes: every routed expert's codes and scales once,
    x and out."""
    import torch
    import knurlogic_amd as KA
    from knurlogic_amd import nn
    E, k, H, I = MOE["E"], MOE["k"], MOE["H"], MOE["I"]
    bits = 4 if mode == "mxfp4" else 8

    def mat_bytes(N, K):
        return N * (K * bits // 8 + K // 32)

    per_e = 2 * mat_bytes(I, H) + mat_bytes(H, I)
    n = max(4, math.ceil(ROTATE_BYTES / (E * per_e)))
    g = torch.Generator(device=dev).manual_seed(6000 + T)

    def mat(N, K):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, N, K * bits // 32), device=dev, generator=g,
                          dtype=torch.int32).view(torch.uint32)
        sc = torch.randint(118, 124, (E, N, K // 32), device=dev, generator=g, dtype=torch.int32).to(torch.uint8)
        return nn.QuantizedSwitchLinear(w, sc, None, None, 32, bits, mode)

    glus = [nn.SwitchGLU(mat(I, H), mat(I, H), mat(H, I)) for _ in range(n)]
    x = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, device=dev, generator=g).to(torch.bfloat16)
    inds, _ = KA.moe_route(logits, k)
    distinct = int(torch.unique(inds).numel())

    def run():
        for i in range(calls):
            ii, sc = KA.moe_route(logits, k)
            glus[i % n].combine(x, ii, sc)

    us = time_graph(run) / calls * 1e3
    nbytes = distinct * per_e + 2 * 2 * T * H
    gbs = nbytes / (us * 1e-6) / 1e9
    del glus
    torch.cuda.empty_cache()
    return {"op": f"{mode}_moe_experts", "T": T, "experts_routed": distinct, "cache": "cold",
            "us": round(us, 3), "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "bound": "hbm", "bytes": nbytes, "flops": 2.0 * T * k * 3 * H * I}


def bench_mx_dense(mode, M, N, K, calls, dev):
    """quantized_matmul over a microscaled weight [N, K] (mxfp4: E2M1 codes,
    mxfp8: E4M3; one E8M0 scale byte per 32 inputs, no biases), weight sets
    rotated past 1 GB.  Bytes: codes and scales once, x and y."""
    import torch
    import knurlogic_amd as KA
    bits = 4 if mode == "mxfp4" else 8
    per = N * (K * bits // 8 + K // 32)
    n = max(4, math.ceil(ROTATE_BYTES / per))
    g = torch.Generator(device=dev).manual_seed(7000 + M)
    sets = []
    for _ in range(n):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K * bits // 32), device=dev, generator=g,
                          dtype=torch.int32).view(torch.uint32)
        sc = torch.randint(118, 124, (N, K // 32), device=dev, generator=g, dtype=torch.int32).to(torch.uint8)
        sets.append((w, sc))
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)

    def run():
        for i in range(calls):
            w, sc = sets[i % n]
            KA.quantized_matmul(x, w, sc, None, True, 32, bits, mode)

    us = time_graph(run) / calls * 1e3
    nbytes = per + 2 * M * K + 2 * M * N
    gbs = nbytes / (us * 1e-6) / 1e9
    del sets
    torch.cuda.empty_cache()
    return {"op": f"{mode}_quantized_matmul", "M": M, "N": N, "K": K, "cache": "cold", "us": round(us, 3),
            "GBps": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm", "bytes": nbytes,
            "flops": 2.0 * M * N * K}


def ceilings(dev, headline_bytes):
    """Measured ceilings beside the published peaks: the HBM read rate of a
    plain read kernel (kmi_read_probe, 16-byte nontemporal loads, nothing
    computed) over the headline's per-call bytes with the buffers rotated
    past the Infinity Cache as the headline's are, over the [4096, 4096]
    M = 1 call's bytes, over 64 KB (one launch's floor) and over 1 GiB; the
    bf16 MFMA rate and clock of the GEMM's matrix-core work alone
    (mfma_rate); and the bf16 GEMM rate of torch.matmul (hipBLASLt) on the
    prefill shapes with unquantized bf16 weights."""
    import ctypes
    import torch
    from knurlogic_amd import _abi
    L = _abi.load()
    out = torch.zeros(1, dtype=torch.int32, device=dev)

    def read_rate(nbytes, wgs):
        nbytes = nbytes // 16 * 16
        n = max(4, math.ceil(ROTATE_BYTES / nbytes))
        bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(n)]
        calls = max(n, 40)

        def run():
            st = torch.cuda.current_stream().cuda_stream
            for i in range(calls):
                _abi.check(L.kmi_read_probe(ctypes.c_void_p(bufs[i % n].data_ptr()), nbytes, wgs,
                                            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st)), "read_probe")

        us = time_graph(run) * 1e3 / calls
        del bufs
        torch.cuda.empty_cache()
        return nbytes / (us * 1e-6) / 1e9, us

    res = {}
    best = max((read_rate(headline_bytes, w) + (w,) for w in (512, 1024, 2048, 4096)), key=lambda t: t[0])
    res["read_headline_bytes"] = {"bytes": headline_bytes // 16 * 16, "GBps": round(best[0], 1),
                                  "us": round(best[1], 3), "workgroups": best[2],
                                  "frac_of_published": round(best[0] / PEAK_HBM_GBS, 4)}
    # the [4096, 4096] M = 1 call's bytes, and the floor of one launch in a
    # graph (64 KB read by 256 workgroups)
    b4k = dense_bytes(1, 4096, 4096, 4)
    best1 = max((read_rate(b4k, w) + (w,) for w in (256, 512, 1024, 2048)), key=lambda t: t[0])
    res["read_4096x4096_m1_bytes"] = {"bytes": b4k // 16 * 16, "GBps": round(best1[0], 1),
                                      "us": round(best1[1], 3), "workgroups": best1[2],
                                      "frac_of_published": round(best1[0] / PEAK_HBM_GBS, 4)}
    res["launch_floor_us"] = round(read_rate(1 << 16, 256)[1], 3)
    big = max((read_rate(1 << 30, w) + (w,) for w in (2048, 8192)), key=lambda t: t[0])
    res["read_1GiB"] = {"GBps": round(big[0], 1), "us": round(big[1], 3), "workgroups": big[2],
                        "frac_of_published": round(big[0] / PEAK_HBM_GBS, 4)}
    res["mfma_bf16"] = mfma_rate(dev, L)
    for N, K in ((14336, 4096), (4096, 14336)):
        g = torch.Generator(device=dev).manual_seed(N)
        x = torch.randn(512, K, device=dev, generator=g).to(torch.bfloat16)
        w = torch.randn(K, N, device=dev, generator=g).to(torch.bfloat16)     # [K, N]: no transposed view
        y = torch.empty(512, N, device=dev, dtype=torch.bfloat16)
        calls = 30

        def mm():
            for _ in range(calls):
                torch.matmul(x, w, out=y)

        us = time_graph(mm) * 1e3 / calls
        tf = 2.0 * 512 * N * K / (us * 1e-6) / 1e12
        res[f"bf16_gemm_512x{N}x{K}"] = {"us": round(us, 3), "TFLOPs": round(tf, 1),
                                        "frac_of_published": round(tf / PEAK_BF16_TFLOPS, 4),
                                        "what": "torch.matmul bf16 (hipBLASLt), unquantized weights, warm"}
        del x, w, y
    torch.cuda.empty_cache()
    return res


def mfma_rate(dev, L=None, rounds=2048):
    """The bf16 MFMA rate the matrix cores reach on the prefill GEMM's
    instruction and wave layout alone (kmi_mfma_probe: one workgroup of 8
    waves per CU, 16 v_mfma_f32_32x32x16_bf16 per wave per round on register
    operands), and the shader clock under that load from the probe's cycle
    and 100 MHz counters; peak_at_clock is 1024 FLOPs per SIMD per cycle at
    that clock."""
    import ctypes
    import torch
    from knurlogic_amd import _abi
    L = L or _abi.load()
    ncu = torch.cuda.get_device_properties(dev).multi_processor_count
    seed = torch.full((64,), 0x3C003C00, dtype=torch.int32, device=dev)     # bf16 pairs of 2^-7
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    stamps = torch.zeros(2, dtype=torch.int64, device=dev)
    calls = 4

    def run():
        st = torch.cuda.current_stream().cuda_stream
        for _ in range(calls):
            _abi.check(L.kmi_mfma_probe(ctypes.c_void_p(seed.data_ptr()), ncu, rounds, ctypes.c_void_p(out.data_ptr()),
                                        ctypes.c_void_p(stamps.data_ptr()), ctypes.c_void_p(st)), "mfma_probe")

    us = time_graph(run) * 1e3 / calls
    flops = ncu * 8 * rounds * 16 * 2.0 * 32 * 32 * 16
    tf = flops / (us * 1e-6) / 1e12
    cyc, ticks = (int(v) for v in stamps.cpu())
    mhz = cyc * 100.0 / ticks if ticks > 0 else None
    return {"TFLOPs": round(tf, 1), "us": round(us, 3), "workgroups": ncu, "frac_of_published": round(tf / PEAK_BF16_TFLOPS, 4),
            "clock_MHz": round(mhz, 0) if mhz else None,
            "peak_at_clock_TFLOPs": round(ncu * 4 * 1024 * mhz * 1e6 / 1e12, 1) if mhz else None,
            "what": "kmi_mfma_probe: v_mfma_f32_32x32x16_bf16 on register operands, 8 waves per CU"}


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


HEADLINE_PROFILE = ROOT / "profiles" / "qmv_4bit_14336x4096_m1.md"


def profiled_traffic():
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by a known-size copy);
    None when the summary is absent."""
    try:
        for line in HEADLINE_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        return None
    return None


def cpu_baseline(seconds=10.0):
    """The oracle's quantized_matmul (C, OpenMP) on this host's cores, 4-bit
    M=1 [14336, 4096]: calls repeated until ~`seconds` of wall time."""
    import numpy as np
    import oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rng = np.random.default_rng(0)
    N, K = 14336, 4096
    w = O.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    wq, s, b = O.quantize(w, 64, 4)
    x = O.bf16_round(rng.standard_normal((1, K)).astype(np.float32))
    O.quantized_matmul(x, wq, s, b, True, 64, 4, "bfloat16", threads)   # warm
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.quantized_matmul(x, wq, s, b, True, 64, 4, "bfloat16", threads)
        n += 1
    dt = (time.perf_counter() - t0) / n
    gbs = dense_bytes(1, N, K, 4) / dt / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "us_per_call": round(dt * 1e6, 1),
            "sample": f"oracle quantized_matmul (C/OpenMP, float64 accumulate), 4-bit g64 "
                      f"[14336,4096] M=1, {n} calls in {seconds:.0f} s"}


#: the headline step: one decode token through a stack of this many layers,
#: each a [14336, 4096] 4-bit GEMV over its own weight (a Llama-3-8B-sized
#: MLP projection per layer; the weight sets rotate past 1 GB, so every
#: layer's weight comes from HBM)
LAYERS_PER_STEP = 32


def _pct(r):
    if r.get("bound") == "mfma":
        return f"{100 * r['mfma_frac']:.1f}%mfma"
    return f"{100 * r['hbm_frac']:.1f}%hbm"


def summary(detail):
    """One short string per workload row (cold where both were measured):
    workload and shape, µs per call and % of the bounding peak.  Printed
    last in the JSON line."""
    out = {}
    for r in detail:
        if r.get("cache") == "warm":
            continue
        op = r["op"]
        if op == "quantized_matmul":
            if (r["N"], r["K"]) == (4096, 4096):
                key = f"gemv {r['bits']}b 4096x4096 M{r['M']}"
            else:
                key = f"qmm {r['bits']}b {r['N']}x{r['K']} M{r['M']}"
        elif op == "moe_experts":
            key = f"moe T{r['T']}" if r["T"] <= 256 else f"prefill moe T{r['T']}"
        elif op == "vq_moe_experts":
            key = (f"vq {r['codebook'].split()[0]} T{r['T']}" if r["T"] <= 16
                   else f"prefill vq {r['codebook'].split()[0]} T{r['T']}")
        elif op == "kv8_decode":
            key = f"kv8 {r['N'] // 1024}k L{r['L']}" + (f" D{r['D']} R{r['H'] // r['Hk'] * r['L']}"
                                                          if r["D"] != 128 else "")
        else:
            continue
        out[key] = f"{r['us']}us {_pct(r)}"
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # steps of LAYERS_PER_STEP calls each, all in one HIP graph: the graph
    # launch's fixed start-up (measured +0.3-0.4 us per call when spread over
    # 200 calls) is spread over steps x 32 calls
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline only, no detail table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="detail sections, comma-separated "
                                                "(gemv4k, dense, kv8, kvcache, qsdpa, moe, vq; gemv4k = the "
                                                "[4096, 4096] M = 1 rows alone); default all")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the measured read and bf16 GEMM ceilings")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 10 plain device copies of MIB MiB (the known-size kernel "
                         "that calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.copy_probe:
        import torch
        n = args.copy_probe << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": 10}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the path is not sharded "
                          "and no figure at several GPUs exists (bench.py --gpus 1)"}))
        sys.exit(2)

    import torch
    import knurlogic_amd as KA
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bits, M, N, K = 4, 1, 14336, 4096
    Lps = LAYERS_PER_STEP

    # headline: W untimed steps eagerly, then one graph of exactly K steps
    # (K x 32 layer calls)
    sets = make_sets(N, K, bits, True, dev)
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    for i in range(args.warmup * Lps):
        KA.quantized_matmul(x, *sets[i % len(sets)], transpose=True, group_size=64, bits=bits)
    torch.cuda.synchronize()

    def run():
        for i in range(args.steps * Lps):
            wq, s, b = sets[i % len(sets)]
            KA.quantized_matmul(x, wq, s, b, transpose=True, group_size=64, bits=bits)

    # untimed replays first (the GPU leaves its idle clocks), then exactly
    # `steps` steps timed
    ms_total = time_graph(run, replays=1, warm=4)
    del sets
    torch.cuda.empty_cache()
    ms_step = ms_total / args.steps
    us = ms_step * 1e3 / Lps                       # per layer call
    nbytes = dense_bytes(M, N, K, bits)
    gbs = nbytes / (us * 1e-6) / 1e9

    detail = []
    only = set(args.only.split(",")) if args.only else {"gemv4k", "dense", "kv8", "kvcache", "qsdpa", "moe", "vq"}
    full = not args.quick
    # the dense configurations (1, 2) first; the MoE, VQ and KV8 rows
    # (configurations 3-5) last, so they end the line
    if full and ("gemv4k" in only or "dense" in only):
        detail.append(bench_dense(4, 1, 4096, 4096, True, 200, dev))
        detail.append(bench_dense(4, 1, 4096, 4096, False, 200, dev))
    if full and "dense" in only:
        for b_ in (4, 8):
            for shape in ((14336, 4096), (4096, 14336)):
                for m in (1, 16, 512):
                    for cold in (True, False):
                        calls = 100 if m < 512 else 30
                        detail.append(bench_dense(b_, m, shape[0], shape[1], cold, calls, dev))
        for mode in ("mxfp4", "mxfp8"):
            for m in (1, 16):
                detail.append(bench_mx_dense(mode, m, 14336, 4096, 100, dev))
    if full and "kvcache" in only:
        for s_ in (1, 512):
            detail.append(bench_kv_append(4, 4, s_, 128, 8, 200 if s_ == 1 else 50, dev))
    if full and "qsdpa" in only:
        for n_ in (8192, 32768):
            for l_ in (1, 4):
                detail.append(bench_qsdpa(4, 32, 4, l_, n_, 128, 8, 30, dev))
    if full and "vq" in only:
        for t_ in (1, 16):
            detail.append(bench_vq_packed(t_, 50, dev))
        for t_ in (1, 16):      # the shipped Gemma-4 26B VQ artifact's expert shape
            detail.append(bench_vq_packed(t_, 50, dev, dim=2, H=2816, I=704))
    if full and "moe" in only:
        for t_ in (1, 16):
            detail.append(bench_mx_moe(t_, 30, dev))
        for t_ in (512, 2048):             # prefill chunks (not a decode-step row)
            detail.append(bench_moe(t_, True, 5, dev))
    if full and "vq" in only:
        for kc_ in (256, 4096):
            for t_ in (512, 2048):         # prefill chunks (not a decode-step row)
                detail.append(bench_vq(t_, kc_, True, 5, dev))
    if full and "moe" in only:
        for t_ in (1, 16, 256):
            for cold in (True, False):
                detail.append(bench_moe(t_, cold, 50 if t_ < 256 else 20, dev))
    if full and "vq" in only:
        for kc_ in (256, 4096):
            for t_ in (1, 16):
                for cold in (True, False):
                    detail.append(bench_vq(t_, kc_, cold, 50, dev))
    if full and "kv8" in only:
        for n_ in (8192, 32768):
            for l_ in (1, 4):
                for cold in (True, False):
                    detail.append(bench_kv8(4, 32, 4, l_, n_, 128, cold, 50, dev))
        # head dims 256 and 512 (16 query heads over 4 KV heads), and 64 query
        # rows per KV head at 512 (16 heads over 1, 4 tokens): cold only
        for h_, hk_, l_, d_ in ((16, 4, 1, 256), (16, 4, 1, 512), (16, 1, 4, 512)):
            detail.append(bench_kv8(4, h_, hk_, l_, 32768, d_, True, 20, dev))

    ceil = None if (args.quick or args.no_ceilings) else ceilings(dev, nbytes)
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u4",
        "data": "synthetic: W ~ N(0, 0.02) quantized on the GPU (affine, 4-bit, group 64), "
                "x ~ N(0, 1) bf16",
        "config": {"workload": "affine 4-bit g64 quantized_matmul, W [14336,4096], M=1 "
                               "(decode GEMV), bf16 activations, fp32 accumulate; one step = one "
                               f"decode token through {Lps} layers, each its own weight",
                   "layers_per_step": Lps, "bytes_per_step": nbytes * Lps,
                   "us_per_layer": round(us, 3), "cache": "cold (weight sets rotated past 1 GB)",
                   "device": torch.cuda.get_device_name(dev)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": profiled_traffic(),
                     "algorithmic_bytes": nbytes, "launch_us": round(us, 3),
                     "traffic_source": "profiles/qmv_4bit_14336x4096_m1.md",
                     "measured_read_ceiling": (ceil or {}).get("read_headline_bytes")},
        "ceilings": ceil,
        "cpu_baseline": cpu,
        "detail": detail,
        "summary": summary(detail),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
