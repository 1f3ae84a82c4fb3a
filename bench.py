"""Decode throughput on the Gemma-2-2B shape on one MI355X.

A step is one greedy decode token through the whole model: embedding, 26
layers of RMSNorm -> QKV matvec -> KV-cache write -> split-KV FlashDecoding
-> O projection -> residual, gated MLP -> residual, then the final norm,
the tied LM head (256000 x 2304) and argmax. Weights are random N(0, 0.02)
bf16 filled on the device, the KV cache holds 4096 synthetic N(0, 1) rows,
and the timed steps decode positions 4096, 4097, ... from a prompt token
drawn uniformly from the vocabulary (seed 0). Steps replay a captured HIP
graph of `graph_steps` tokens; inputs are resident in HBM before timing.

Besides the JSON line's throughput it reports, per kernel, the mean launch
time measured with HIP events with the kernel launched alone over every
layer's weights, its algorithmic bytes and the fraction of the 8 TB/s HBM
peak; `roofline` is the dominant kernel (the fused gate/up matvec).
`cpu_baseline` is the CPU oracle (scalar C, one core) timed on a bounded
sample of the same decode: a few layers' steps plus the LM head, scaled to
26 layers.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
START_POS = 4096


def kernel_bytes(cfg, name, pos):
    """Algorithmic HBM bytes of one launch of `name` in a decode step at `pos`."""
    H, F, V = cfg.hidden, cfg.ffn, cfg.vocab
    QW, KW = cfg.query_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    QKV = QW + 2 * KW
    if name.startswith("gated_mlp_gate_up"):  # residual + norm, Wg and Wu, h
        return 2 * F * H * 2 + 3 * H * 2 + 2 * H * 4 + F * 2
    if name == "matvec_nk_stream_bf16_bf16_bf16_r1":  # down projection (K = F)
        return H * F * 2 + F * 2 + H * 2
    if name in ("decode_matvec_bf16_bf16_r1_f2", "decode_matvec_bf16_bf16_r1_f3"):  # QKV (+ residual), norm, KV scatter
        return QKV * H * 2 + 3 * H * 2 + 2 * H * 4 + QKV * 2
    if name == "decode_matvec_bf16_bf16_r1_f0":  # output projection (K = QW)
        return H * QW * 2 + QW * 2 + H * 2
    if name == "decode_matvec_bf16_f32_r4_f3":  # residual, final norm, LM head
        return V * H * 2 + 3 * H * 2 + 2 * H * 4 + V * 4
    if name.startswith("flash_decoding_partial"):
        return 2 * KW * (pos + 1) * 2 + 2 * QW * 2  # K and V rows + q
    if name.startswith("flash_decoding_fresh"):  # K and V rows, raw q/k/v, new K/V row, norm weights
        return 2 * KW * pos * 2 + QKV * 2 + 2 * KW * 2 + 2 * cfg.head_dim * 4
    # 4-bit weights (group 64): 0.5 byte per weight + a bf16 scale and bias per group
    q4 = lambda n, k: n * k // 2 + n * (k // 64) * 4
    if name.startswith("q4_gate_up_bf16_l") and name.endswith("_res"):
        return 2 * q4(F, H) + 3 * H * 2 + 2 * H * 4 + F * 2
    if name.startswith("q4_decode_matvec_bf16_bf16_l") and name.endswith(("_f2", "_f3")):
        return q4(QKV, H) + 3 * H * 2 + 2 * H * 4 + QKV * 2
    if name.startswith("q4_decode_matvec_bf16_bf16_l") and name.endswith("_f0"):
        return q4(H, QW) + QW * 2 + H * 2
    if name.startswith("q4_decode_matvec_bf16_f32_l") and name.endswith("_f3"):
        return q4(V, H) + 3 * H * 2 + 2 * H * 4 + V * 4
    if name.startswith("aq_qmv_fast_bf16_bf16_bf16_b4_g64_l") and name.endswith("_j8"):  # down (K = F)
        return q4(H, F) + F * 2 + H * 2
    return None


def cpu_baseline(dec, cfg, stream, token, layers_sample=3, steps_sample=2):
    """The oracle (scalar C, one thread) on a bounded sample of the decode:
    `steps_sample` tokens through `layers_sample` layers, plus one LM head,
    both on this decoder's weights; tok/s extrapolated to all layers."""
    import oracle as O

    BF = O.BF16

    def host(name, layer=0):
        t = dec.tensor(name, layer)
        raw = t.numpy(stream)
        return raw if t.dtype == "f32" else O.from_bits(raw.view(np.uint16), BF)

    H = cfg.hidden
    names = [("in_norm", "norm_in"), ("qkv", "w_qkv"), ("o", "w_o"), ("post_attn_norm", "norm_post_attn"),
             ("pre_ffn_norm", "norm_pre_ffn"), ("gate", "w_gate"), ("up", "w_up"), ("down", "w_down"),
             ("post_ffn_norm", "norm_post_ffn")]
    W = [{n: host(t, l) for n, t in names} for l in range(layers_sample)]
    caches = [(host("k_cache", l)[0].copy(), host("v_cache", l)[0].copy()) for l in range(layers_sample)]
    emb = host("embedding")
    x = O.round_to(O.scalar_mul(emb[token], float(np.sqrt(np.float32(H)))), BF)
    # one core: the reference's CPU loops are single-threaded scalar code
    # (KernelsTests.swift:239-267); pinned in this process, restored after
    allowed = os.sched_getaffinity(0)
    core = min(allowed)
    os.sched_setaffinity(0, {core})
    try:
        t0 = time.perf_counter()
        for s in range(steps_sample):
            for l in range(layers_sample):
                O.decoder_layer(W[l], x, caches[l][0], caches[l][1], START_POS + s, H=H, Nq=cfg.query_heads,
                                Nkv=cfg.kv_heads, Hd=cfg.head_dim, F=cfg.ffn, eps=cfg.eps, scale=cfg.attn_scale,
                                act_tag=BF)
        t_layers = (time.perf_counter() - t0) / (steps_sample * layers_sample)
        n = O.round_to(O.rmsnorm(x, host("final_norm"), cfg.eps), BF)
        t0 = time.perf_counter()
        logits = O.matmul(n, emb, 1, H, cfg.vocab, True)
        O.argmax(logits)
        t_head = time.perf_counter() - t0
    finally:
        os.sched_setaffinity(0, allowed)
    sec_per_token = cfg.layers * t_layers + t_head
    return {"value": 1.0 / sec_per_token, "unit": "tok/s", "cores": 1, "kind": "port",
            "host": {"cpu": cpu_model(), "nproc": os.cpu_count(), "cores_allowed": len(allowed), "pinned_to": core},
            "sample": (f"oracle decode of {steps_sample} tokens through {layers_sample} of {cfg.layers} layers at "
                       f"ctx {START_POS} ({t_layers * 1e3:.0f} ms/layer) + 1 LM head ({t_head * 1e3:.0f} ms), "
                       f"scaled to {cfg.layers} layers, on one core")}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic(name):
    """HBM bytes per launch of `name` from the committed rocprofv3 --pmc summary."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return t.get(name, {}).get("bytes_per_launch")


def copy_calibration(pa, nbytes=1 << 30, copies=3):
    """A plain copy of known size: its per-dispatch FETCH_SIZE and WRITE_SIZE
    (KiB) against `nbytes` give the scale of those counters on this GPU."""
    from popcorn_amd import runtime as R

    src, dst = pa.DeviceBuffer(nbytes), pa.DeviceBuffer(nbytes)
    stream = pa.Stream()
    h = R._stream_handle(stream)
    R.check(R.lib().popcorn_memset(src.ptr, 1, nbytes, h))
    for _ in range(copies):
        R.check(R.lib().popcorn_memcpy_d2d(dst.ptr, src.ptr, nbytes, h))
    stream.synchronize()
    print(json.dumps({"calibration": "device-to-device copy", "bytes": nbytes, "copies": copies}))


def timed_launches(pa, stream, enc, kerns):
    """Mean microseconds per launch of `kerns`, enqueued by one native call
    (no Python between launches) between two events on `stream`."""
    e0, e1 = pa.Event(), pa.Event()
    e0.record(stream)
    enc.encode(*kerns)
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_ms(e1) * 1e3 / len(kerns)


def q4_sweep(pa, lib, stream, enc):
    """The 4-bit decode matvec (aq_qmv_fast, bf16 x, bf16 scales and biases,
    group 64) at the Gemma-2-2B decode shapes; every launch reads a weight set
    it has not read for >= 512 MB of others (cold in the MALL). Bytes: packed
    words + scales + biases + x + y."""
    rows = []
    for name, N, K in (("qkv", 4096, 2304), ("o_proj", 2304, 2048), ("gate_or_up", 9216, 2304),
                       ("down", 2304, 9216), ("lm_head", 256000, 2304)):
        wbytes = N * K // 2 + 2 * N * (K // 64) * 2
        nbytes = wbytes + K * 2 + N * 2
        sets = max(1, min(64, -(-(512 << 20) // wbytes)))
        packed = pa.Tensor.empty([sets * N * K // 8], "u32")
        scales = pa.Tensor.empty([sets * N * (K // 64)], "bf16")
        biases = pa.Tensor.empty([sets * N * (K // 64)], "bf16")
        lib.fill_normal(packed.view([sets * N * K // 8], "f32"), 1, stream=stream)
        lib.fill_normal(scales, 2, std=0.01, stream=stream)
        lib.fill_normal(biases, 3, std=0.01, stream=stream)
        x = pa.Tensor.empty([1, K], "bf16")
        lib.fill_normal(x, 4, stream=stream)
        y = pa.Tensor.empty([1, N], "bf16")
        qts = [pa.AffineQuantizedTensor(packed.view([N, K // 8], offset_elements=i * N * K // 8),
                                        scales.view([N, K // 64], offset_elements=i * N * (K // 64)),
                                        biases.view([N, K // 64], offset_elements=i * N * (K // 64)), [N, K])
               for i in range(sets)]
        kerns = [pa.Kernels.Matmul(x, q, y) for q in qts]
        reps = max(sets, min(512, int(4e9 // nbytes)))
        enc.encode(*kerns)
        stream.synchronize()
        us = timed_launches(pa, stream, enc, [kerns[r % sets] for r in range(reps)])
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"matvec": name, "N": N, "K": K, "kernel": kerns[0].function_names[0], "us": round(us, 2),
                     "bytes": nbytes, "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3)})
        del kerns, qts, packed, scales, biases
    return rows


def q4_prompt_gemm(pa, lib, stream, enc, reps=10):
    """The 4-bit Matmul for a prompt (bf16 x, bf16 scales and biases, group
    64) at the Gemma-2-2B gate and down shapes: m = 2048 and 128 rows on the
    matrix-core GEMM (aq_gemm.hip; prep, GEMM or split GEMM + reduction,
    all timed), beside the streaming matvec per row the reference's route
    runs (Matmul.swift:279-332), timed at m = 15 (its largest m here) and
    reported per row. TFLOP/s count 2 m N K; frac is of the dense bf16 peak."""
    rows = []
    for name, N, K in (("gate", 9216, 2304), ("down", 2304, 9216)):
        packed = pa.Tensor.empty([N, K // 8], "u32")
        scales, biases = pa.Tensor.empty([N, K // 64], "bf16"), pa.Tensor.empty([N, K // 64], "bf16")
        lib.fill_normal(packed.view([N * K // 8], "f32"), 6, stream=stream)
        lib.fill_normal(scales, 7, std=0.01, stream=stream)
        lib.fill_normal(biases, 8, std=0.01, stream=stream)
        qt = pa.AffineQuantizedTensor(packed, scales, biases, [N, K])
        out = {}
        for m in (15, 128, 2048):
            x = pa.Tensor.empty([m, K], "bf16")
            lib.fill_normal(x, 9, stream=stream)
            y = pa.Tensor.empty([m, N], "bf16")
            k = pa.Kernels.Matmul(x, qt, y)
            enc.encode(k)
            stream.synchronize()
            us = timed_launches(pa, stream, enc, [k] * reps)
            tf = 2.0 * m * N * K / (us * 1e-6) / 1e12
            out[f"m{m}"] = {"kernels": k.function_names, "us": round(us, 1), "TFLOP_s": round(tf, 1),
                            "frac": round(tf / MFMA_PEAK_F16_TFLOPS, 3)}
        out["per_row_us_per_row"] = round(out["m15"]["us"] / 15, 2)
        out["m2048_speedup_vs_per_row"] = round(out["per_row_us_per_row"] * 2048 / out["m2048"]["us"], 1)
        rows.append({"matmul": name, "N": N, "K": K, **out})
    return rows


def skinny_gemm(pa, lib, stream, enc):
    """The skinny 16-bit Matmul (2 <= M <= 64; the reference's small-M MPP
    tiles, Matmul.swift:175-196): C[M, N] = A[M, K] . B[N, K]^T in bf16 with
    f32 accumulation at M = 8 on the Gemma-2-2B gate shape (N 9216, K 2304:
    an 8-token prompt or an 8-wide decode batch) and at M = 16, 32, 64; every
    launch reads a B it has not read for >= 512 MB of others (cold in the
    MALL). Bytes: B + A + C."""
    rows = []
    N, K = 9216, 2304
    wbytes = N * K * 2
    sets = max(1, -(-(512 << 20) // wbytes))
    w = pa.Tensor.empty([sets * N, K], "bf16")
    lib.fill_normal(w, 5, std=0.02, stream=stream)
    for M in (8, 16, 32, 64):
        a = pa.Tensor.empty([M, K], "bf16")
        lib.fill_normal(a, 6, stream=stream)
        c = pa.Tensor.empty([M, N], "bf16")
        kerns = [pa.Kernels.Matmul(a, w.view([N, K], offset_elements=i * N * K), c, True) for i in range(sets)]
        enc.encode(*kerns)
        stream.synchronize()
        nbytes = wbytes + M * K * 2 + M * N * 2
        us = timed_launches(pa, stream, enc, [kerns[r % sets] for r in range(8 * sets)])
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"M": M, "N": N, "K": K, "kernel": kerns[0].function_names[0], "us": round(us, 2),
                     "bytes": nbytes, "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3),
                     "TFLOP_s": round(2 * M * N * K / (us * 1e-6) / 1e12, 2)})
    del w
    return rows


def fd_sweep(pa, lib, stream, enc):
    """split-KV FlashDecoding (partial + LSE combine) in f16,
    Q [B, 8, 1, 256], K/V [B, 4, ctx, 256] N(0, 1), scale 1/16, no mask, over
    B x ctx. Every launch reads a KV set it has not read for >= 512 MB of other
    sets (cold in the 256 MB MALL), so the rate is HBM's."""
    out_rows = []
    for B in (1, 8, 32):
        for ctx in (2048, 8192, 32768):
            kv_elems = B * 4 * ctx * 256
            nbytes = 2 * kv_elems * 2 + 2 * B * 8 * 256 * 2
            sets = max(1, min(64, -(-(512 << 20) // (2 * kv_elems * 2))))
            kpool = pa.Tensor.empty([sets * kv_elems], "f16")
            vpool = pa.Tensor.empty([sets * kv_elems], "f16")
            lib.fill_normal(kpool, 1, stream=stream)
            lib.fill_normal(vpool, 2, stream=stream)
            q = pa.Tensor.empty([B, 8, 1, 256], "f16")
            lib.fill_normal(q, 3, stream=stream)
            o = pa.Tensor.empty([B, 8, 1, 256], "f16")
            kerns = [pa.Kernels.FlashAttention(q, kpool.view([B, 4, ctx, 256], offset_elements=i * kv_elems),
                                               vpool.view([B, 4, ctx, 256], offset_elements=i * kv_elems), o,
                                               scale=1 / 16, mask=pa.AttentionMask(2), batch=B, query_heads=8,
                                               kv_heads=4, query_len=1, key_len=ctx, head_dim=256)
                     for i in range(sets)]
            reps = max(3, sets, min(256, int(4e9 // nbytes)))
            enc.encode(*kerns)
            stream.synchronize()
            us = timed_launches(pa, stream, enc, [kerns[r % sets] for r in range(reps)])
            gbs = nbytes / (us * 1e-6) / 1e9
            out_rows.append({"B": B, "ctx": ctx, "launches": reps, "us": round(us, 2), "GB_s": round(gbs, 1),
                             "frac": round(gbs / HBM_PEAK_GBS, 3)})
            del kerns, kpool, vpool
    return out_rows


def mlp_config3(pa, lib, stream, enc, sets=4, reps=64):
    """the Gemma-2B-shaped MLP decode at batch 1 in bf16
    (f32 accumulation): RMSNorm over x [2304] (N(0, 1), eps 1e-6, weight
    1 + N(0, 0.1)), the fused gate/up matvec ([9216, 2304] each, N(0, 0.02))
    with GELU-tanh gating, then the down matvec ([2304, 9216]). `sets` weight
    sets (510 MB, cold in the 256 MB MALL) are cycled. Bytes: the three
    matrices, x, the norm weight, the hidden vector written and read, y."""
    H, F = 2304, 9216
    x = pa.Tensor.empty([H], "bf16")
    lib.fill_normal(x, 61, stream=stream)
    nw = pa.Tensor.empty([H], "f32")
    lib.fill_normal(nw, 62, mean=1.0, std=0.1, stream=stream)
    wg = pa.Tensor.empty([sets * F * H], "bf16")
    wu = pa.Tensor.empty([sets * F * H], "bf16")
    wd = pa.Tensor.empty([sets * H * F], "bf16")
    for i, w in enumerate((wg, wu, wd)):
        lib.fill_normal(w, 63 + i, std=0.02, stream=stream)
    y = pa.Tensor.empty([H], "bf16")
    hid = pa.Tensor.empty([F], "bf16")
    kerns = [pa.Kernels.GatedMLP(x, nw, wg.view([F, H], offset_elements=i * F * H),
                                 wu.view([F, H], offset_elements=i * F * H),
                                 wd.view([H, F], offset_elements=i * H * F), y, eps=1e-6, hidden=hid)
             for i in range(sets)]
    enc.encode(*kerns)
    stream.synchronize()
    us = timed_launches(pa, stream, enc, [kerns[r % sets] for r in range(reps)])
    nbytes = 3 * F * H * 2 + H * 2 + H * 4 + 2 * F * 2 + H * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"kernels": kerns[0].function_names, "us": round(us, 2), "bytes": nbytes, "GB_s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 3)}


MFMA_PEAK_F16_TFLOPS = 2500.0
MFMA_PEAK_F32_TFLOPS = 157.3   # dense f32 on the matrix cores


def prefill_config5(pa, lib, stream, enc, reps=8):
    """BASELINE config 5 (Gemma-7B-shaped single-layer prefill, f16, f32
    accumulation, seq 2048): the QKV Matmul [2048, 3072] x [9216, 3072]^T, the
    MLP Matmuls (gate, up [24576, 3072]; down [3072, 24576]) and causal
    FlashAttention [1, 16, 2048, 256] on the MFMA kernels. Activations N(0, 1),
    weights N(0, 0.02). Each timed over `reps` launches after one warmup.
    The attention is timed before the GEMMs ("attention", the one in
    layer_total) and again after them ("attention_after_gemms"): the GEMMs'
    milliseconds of matrix-core load leave the GPU at a lower clock (power),
    which the attention kernel right after them inherits."""
    S, H, F, QKV = 2048, 3072, 24576, 3 * 3072
    # causal FlashAttention [1, 16, 2048, 256], scale 1/16: 4 flop per (query,
    # key, dim) over the S (S + 1) / 2 unmasked pairs of each head
    Hq, Hd = 16, 256
    q, k, v, o = (pa.Tensor.empty([1, Hq, S, Hd], "f16") for _ in range(4))
    for i, t in enumerate((q, k, v)):
        lib.fill_normal(t, 50 + i, stream=stream)
    fa = pa.Kernels.FlashAttention(q, k, v, out=o, scale=1 / 16, batch=1, query_heads=Hq, kv_heads=Hq,
                                   query_len=S, key_len=S, head_dim=Hd)
    fa_flop = 4.0 * Hq * Hd * S * (S + 1) / 2

    def time_attention():
        enc.encode(fa)
        stream.synchronize()
        e0, e1 = pa.Event(), pa.Event()
        e0.record(stream)
        for _ in range(reps):
            enc.encode(fa)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        return {"kernel": fa.function_names[0], "us": round(us, 1),
                "TFLOP_s": round(fa_flop / (us * 1e-6) / 1e12, 1),
                "frac": round(fa_flop / (us * 1e-6) / 1e12 / MFMA_PEAK_F16_TFLOPS, 3)}

    rows = {"attention": time_attention()}
    x = pa.Tensor.empty([S, H], "f16")
    h = pa.Tensor.empty([S, F], "f16")
    lib.fill_normal(x, 21, stream=stream)
    lib.fill_normal(h, 22, stream=stream)
    shapes = {"qkv": (x, QKV, H), "gate": (x, F, H), "up": (x, F, H), "down": (h, H, F)}
    total_flop, total_us = 0.0, 0.0
    for name, (a, n, k) in shapes.items():
        w = pa.Tensor.empty([n, k], "f16")
        lib.fill_normal(w, 30 + len(rows), std=0.02, stream=stream)
        c = pa.Tensor.empty([S, n], "f16")
        kern = pa.Kernels.Matmul(a, w, c, True)
        enc.encode(kern)
        stream.synchronize()
        e0, e1 = pa.Event(), pa.Event()
        e0.record(stream)
        for _ in range(reps):
            enc.encode(kern)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        flop = 2.0 * S * n * k
        total_flop += flop
        total_us += us
        rows[name] = {"M": S, "N": n, "K": k, "kernel": kern.function_names[0], "us": round(us, 1),
                      "TFLOP_s": round(flop / (us * 1e-6) / 1e12, 1),
                      "frac": round(flop / (us * 1e-6) / 1e12 / MFMA_PEAK_F16_TFLOPS, 3)}
        del w, c, kern
    rows["gemm_total"] = {"us": round(total_us, 1), "TFLOP_s": round(total_flop / (total_us * 1e-6) / 1e12, 1),
                          "frac": round(total_flop / (total_us * 1e-6) / 1e12 / MFMA_PEAK_F16_TFLOPS, 3)}
    rows["attention_after_gemms"] = time_attention()
    total_flop += fa_flop
    total_us += rows["attention"]["us"]
    rows["layer_total"] = {"us": round(total_us, 1), "GFLOP": round(total_flop / 1e9, 1),
                           "TFLOP_s": round(total_flop / (total_us * 1e-6) / 1e12, 1),
                           "frac": round(total_flop / (total_us * 1e-6) / 1e12 / MFMA_PEAK_F16_TFLOPS, 3)}
    return rows


def prefill_attention_hd512(pa, lib, stream, enc, reps=8):
    """Causal FlashAttention at the reference's other matrix-unit bucket,
    head dim 512 (MPPFlashAttention's hd512, FlashAttention.swift:305-311;
    Gemma-4's global layers): [1, 16, 2048, 512] bf16, GQA 2:1, scale
    1/sqrt(512), on the matrix cores; the per-query-row split-KV kernels (the
    route this head dim took before) on the same inputs beside it, reached
    through an output that is not 16-byte aligned."""
    S, Hq, Hkv, Hd = 2048, 16, 8, 512
    q = pa.Tensor.empty([1, Hq, S, Hd], "bf16")
    k, v = (pa.Tensor.empty([1, Hkv, S, Hd], "bf16") for _ in range(2))
    for i, t in enumerate((q, k, v)):
        lib.fill_normal(t, 60 + i, stream=stream)
    o = pa.Tensor.empty([1, Hq, S, Hd + 8], "bf16")
    flop = 4.0 * Hq * Hd * S * (S + 1) / 2
    out = {}
    for name, view in (("tiled", o.view([1, Hq, S, Hd])), ("per_row", o.view([1, Hq, S, Hd], offset_elements=1))):
        fa = pa.Kernels.FlashAttention(q, k, v, out=view, scale=1 / Hd ** 0.5, batch=1, query_heads=Hq,
                                       kv_heads=Hkv, query_len=S, key_len=S, head_dim=Hd)
        enc.encode(fa)
        stream.synchronize()
        e0, e1 = pa.Event(), pa.Event()
        e0.record(stream)
        for _ in range(reps):
            enc.encode(fa)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        out[name] = {"kernel": fa.function_names[0], "us": round(us, 1),
                     "TFLOP_s": round(flop / (us * 1e-6) / 1e12, 1),
                     "frac": round(flop / (us * 1e-6) / 1e12 / MFMA_PEAK_F16_TFLOPS, 3)}
    return out


def prefill_attention_f32(pa, lib, stream, enc, reps=4):
    """Causal FlashAttention in f32 (the reference's mpp_flash_attention_f32,
    FlashAttention.swift:368-376) at the config-5 attention shape,
    [1, 16, 2048, 256], scale 1/16, on v_mfma_f32_16x16x4_f32; the per-row
    split-KV kernels on the same inputs beside it (through an output that is
    not 16-byte aligned). frac is of the f32 matrix-core peak."""
    S, H, Hd = 2048, 16, 256
    q, k, v = (pa.Tensor.empty([1, H, S, Hd], "f32") for _ in range(3))
    for i, t in enumerate((q, k, v)):
        lib.fill_normal(t, 70 + i, stream=stream)
    o = pa.Tensor.empty([1, H, S, Hd + 4], "f32")
    flop = 4.0 * H * Hd * S * (S + 1) / 2
    out = {}
    for name, view in (("tiled", o.view([1, H, S, Hd])), ("per_row", o.view([1, H, S, Hd], offset_elements=1))):
        fa = pa.Kernels.FlashAttention(q, k, v, out=view, scale=1 / 16, batch=1, query_heads=H, kv_heads=H,
                                       query_len=S, key_len=S, head_dim=Hd)
        enc.encode(fa)
        stream.synchronize()
        e0, e1 = pa.Event(), pa.Event()
        e0.record(stream)
        for _ in range(reps):
            enc.encode(fa)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        out[name] = {"kernel": fa.function_names[0], "us": round(us, 1),
                     "TFLOP_s": round(flop / (us * 1e-6) / 1e12, 2),
                     "frac": round(flop / (us * 1e-6) / 1e12 / MFMA_PEAK_F32_TFLOPS, 3)}
    return out


def matmul_forms(pa, lib, stream, enc, reps=5):
    """The reference's other MPP Matmul forms (Matmul.swift:203-214) at
    2048 x 3072 x 3072: a [K, N] bf16 B (transposed into scratch, then the
    MFMA tiles) and f32 output with f32 or mixed f32/bf16 operands (the f32
    matrix-core tiles); frac is of the dense bf16 or f32 matrix-core peak."""
    M, K, N = 2048, 3072, 3072
    out = {}
    for at, bt, ot, tb in (("bf16", "bf16", "bf16", False), ("f32", "f32", "f32", True), ("f32", "f32", "f32", False),
                           ("f32", "bf16", "f32", True), ("bf16", "f32", "f32", False)):
        a = pa.Tensor.empty([M, K], at)
        b = pa.Tensor.empty([N, K] if tb else [K, N], bt)
        c = pa.Tensor.empty([M, N], ot)
        lib.fill_normal(a, 11, stream=stream)
        lib.fill_normal(b, 12, std=0.02, stream=stream)
        k = pa.Kernels.Matmul(a, b, c, tb)
        enc.encode(k)
        stream.synchronize()
        us = timed_launches(pa, stream, enc, [k] * reps)
        tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
        peak = MFMA_PEAK_F16_TFLOPS if (at, bt) == ("bf16", "bf16") else MFMA_PEAK_F32_TFLOPS
        out[f"{at}x{bt}->{ot}" + ("_tb" if tb else "")] = {"kernels": k.function_names, "us": round(us, 1),
                                                            "TFLOP_s": round(tf, 1), "frac": round(tf / peak, 3)}
    return out


def library_reference():
    """The config-5 shapes through the vendor libraries PyTorch calls on ROCm
    (torch.matmul -> hipBLASLt, scaled_dot_product_attention's flash and
    memory-efficient backends), as reference points for the hand-written
    MFMA kernels: same f16 shapes, same FLOP counts. PyTorch carries its own
    HIP runtime, which cannot share a process with this library's, so the
    timing runs in a child process."""
    import subprocess
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--library-reference-child"],
                       capture_output=True, text=True, timeout=900)
    lines = r.stdout.strip().splitlines()
    if r.returncode != 0 or not lines:
        return {"error": (r.stderr.strip().splitlines() or ["no output"])[-1][:200]}
    return json.loads(lines[-1])


def library_reference_child(reps=20):
    import torch
    import torch.nn.functional as Fn

    def timed(f):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            f()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    S, H, F = 2048, 3072, 24576
    out = {"library": f"torch {torch.__version__}"}
    g = torch.Generator(device="cuda").manual_seed(0)
    for name, n, k in (("qkv", 3 * H, H), ("gate", F, H), ("down", H, F)):
        a = torch.randn(S, k, device="cuda", dtype=torch.float16, generator=g)
        w = torch.randn(n, k, device="cuda", dtype=torch.float16, generator=g) * 0.02
        us = timed(lambda: torch.matmul(a, w.t()))
        out[name] = {"us": round(us, 1), "TFLOP_s": round(2.0 * S * n * k / (us * 1e-6) / 1e12, 1)}
        del a, w
    Hq, Hd = 16, 256
    q, k, v = (torch.randn(1, Hq, S, Hd, device="cuda", dtype=torch.float16, generator=g) for _ in range(3))
    flop = 4.0 * Hq * Hd * S * (S + 1) / 2
    from torch.nn.attention import SDPBackend, sdpa_kernel
    for name, be in (("attention_flash", SDPBackend.FLASH_ATTENTION),
                     ("attention_efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel(be):
                us = timed(lambda: Fn.scaled_dot_product_attention(q, k, v, is_causal=True, scale=1 / 16))
            out[name] = {"us": round(us, 1), "TFLOP_s": round(flop / (us * 1e-6) / 1e12, 1)}
        except RuntimeError as ex:  # backend not built for this device
            out[name] = {"error": str(ex)[:120]}
    return out


def time_decode(pa, dec, stream, token, steps, warmup, use_graph):
    """Warmup (captures the graph), then `steps` timed decode steps from the
    same start; seconds, the larger of the wall clock and the HIP events."""
    dec.reset(token, START_POS)
    dec.step(warmup, use_graph=use_graph)
    stream.synchronize()
    dec.reset(token, START_POS)
    pa.synchronize()
    start, stop = pa.Event(), pa.Event()
    t0 = time.perf_counter()
    start.record(stream)
    dec.step(steps, use_graph=use_graph)
    stop.record(stream)
    stop.synchronize()
    pa.synchronize()
    wall = time.perf_counter() - t0
    elapsed = max(wall, start.elapsed_ms(stop) / 1e3)
    tok, pos = dec.read()
    assert pos == START_POS + steps, (pos, steps)
    return elapsed


def decode_variant(pa, lib, stream, D, token, steps, warmup, graph_steps, use_graph, reps, **variant):
    """The config-4 decode with another decoder configuration: tok/s, the HBM
    rate of the whole step, and the mean time of each of the step's kernels.
    attention_block=1: a real attention block (per-head q/k RMSNorm, v RMSNorm,
    RoPE at theta 10000, Gemma4TextInference.swift:352-371) folded into the
    attention partial kernel; weight_bits=4: block-affine 4-bit weights."""
    cfg = D.DecoderConfig(graph_steps=graph_steps, **variant)
    dec = D.Decoder(lib, stream, cfg)
    dec.randomize(seed=0)
    elapsed = time_decode(pa, dec, stream, token, steps, warmup, use_graph)
    names, nd = dec.describe()
    tok_s = steps / elapsed
    step_bytes = dec.step_bytes(int(START_POS + (steps - 1) / 2))
    dec.reset(token, START_POS)
    kernels = {}
    for name in dict.fromkeys(names):
        dec.reset(token, START_POS)
        ms, _ = dec.time_kernel_in_step(name, steps=2)
        kernels[name] = round(ms * 1e3, 2)
    out = {"tok_s": round(tok_s, 2), "ms_per_step": round(elapsed * 1e3 / steps, 4), "dispatches_per_step": nd,
           "hbm_step_GB_s": round(step_bytes * tok_s / 1e9, 1), "kernel_in_step_us": kernels}
    dec.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--graph-steps", type=int, default=8)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=4)
    ap.add_argument("--no-fd-sweep", action="store_true", help="skip the config-2 FlashDecoding sweep")
    ap.add_argument("--no-mlp", action="store_true", help="skip the config-3 MLP decode measurement")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-5 prefill measurement")
    ap.add_argument("--library-reference", action="store_true",
                    help="also time the config-5 shapes through PyTorch's hipBLASLt GEMM and SDPA attention")
    ap.add_argument("--library-reference-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-q4", action="store_true", help="skip the 4-bit matvec measurement")
    ap.add_argument("--no-skinny", action="store_true", help="skip the skinny (2 <= M <= 64) GEMM measurement")
    ap.add_argument("--no-attention-block", action="store_true",
                    help="skip the decode with per-head norms and RoPE (a real attention block)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 3 device-to-device copies of 1 GiB (the known-size kernel that scales the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every GPU box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.library_reference_child:
        print(json.dumps(library_reference_child()))
        return

    import popcorn_amd as pa
    import popcorn_amd.decoder as D

    if pa.device_count() < 1:
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(pa)
        return
    lib = pa.KernelLibrary()
    stream = pa.Stream()
    cfg = D.DecoderConfig(graph_steps=args.graph_steps)
    dec = D.Decoder(lib, stream, cfg)
    dec.randomize(seed=0)
    token = int(np.random.default_rng(0).integers(cfg.vocab))
    use_graph = not args.no_graph
    if START_POS + max(args.steps, args.warmup) > cfg.max_seq:
        raise SystemExit(f"steps above {cfg.max_seq - START_POS} leave the KV cache")

    elapsed = time_decode(pa, dec, stream, token, args.steps, args.warmup, use_graph)
    tokens_per_s = args.steps / elapsed
    mean_pos = START_POS + (args.steps - 1) / 2
    step_bytes = dec.step_bytes(int(mean_pos))

    # per-kernel timing: each kernel alone over all layers' weights, launched
    # back to back from a captured graph; and inside eager steps, as the gap
    # between its end and the end of the launch before it (the kernel after
    # its neighbours, with their cache state; these add up to the step)
    names, nd = dec.describe()
    kernels = {}
    in_step_sum_us = 0.0
    for name in dict.fromkeys(names):
        dec.reset(token, START_POS)
        ims, ilaunches = dec.time_kernel_in_step(name, steps=2)
        in_step_sum_us += ims * 1e3 * names.count(name)
        nbytes = kernel_bytes(cfg, name, START_POS)
        if nbytes is None or ilaunches == 0:
            continue
        igbs = nbytes / (ims * 1e-3) / 1e9
        kernels[name] = {"bytes": nbytes, "in_step_us": round(ims * 1e3, 2), "in_step_GB_s": round(igbs, 1),
                         "in_step_frac": round(igbs / HBM_PEAK_GBS, 3), "in_step_launches": ilaunches}
        if use_graph:  # the back-to-back timing replays a graph (not under --no-graph)
            dec.reset(token, START_POS)
            ms, launches = dec.time_kernel(name, reps=args.kernel_reps)
            gbs = nbytes / (ms * 1e-3) / 1e9
            kernels[name].update({"back_to_back_us": round(ms * 1e3, 2), "back_to_back_frac": round(gbs / HBM_PEAK_GBS, 3),
                                  "back_to_back_launches": launches})
    dec.reset(token, START_POS)
    dominant = "gated_mlp_gate_up_bf16_r1_res"
    dk = kernels[dominant]
    in_step_gbs = dk["bytes"] / (dk["in_step_us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(in_step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(in_step_gbs / HBM_PEAK_GBS, 3), "traffic": load_traffic(dominant),
                "kernel": dominant, "bytes_per_launch": dk["bytes"],
                "timing": "in step: end of each of the kernel's 26 launches minus end of the launch before it (stop events), 2 eager decode steps",
                "mean_us": dk["in_step_us"], "back_to_back_us": dk.get("back_to_back_us"),
                "back_to_back_frac": dk.get("back_to_back_frac")}

    fd = None
    if not args.no_fd_sweep:
        fd = fd_sweep(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))

    mlp = None
    if not args.no_mlp:
        mlp = mlp_config3(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))

    prefill = None
    if not args.no_prefill:
        prefill = prefill_config5(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))
        prefill["attention_hd512"] = prefill_attention_hd512(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))
        prefill["attention_f32"] = prefill_attention_f32(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))
        prefill["matmul_forms"] = matmul_forms(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))
        if args.library_reference:
            prefill["library_reference"] = library_reference()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(dec, cfg, stream, token)

    skinny = None
    if not args.no_skinny:
        skinny = skinny_gemm(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))

    q4 = q4p = None
    if not args.no_q4:
        q4 = q4_sweep(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))
        q4p = q4_prompt_gemm(pa, lib, stream, pa.KernelCommandEncoder(lib, stream))

    block = q4dec = None
    if not args.no_attention_block:
        block = decode_variant(pa, lib, stream, D, token, args.steps, args.warmup, args.graph_steps, use_graph,
                               args.kernel_reps, attention_block=1)
    if not args.no_q4:
        q4dec = decode_variant(pa, lib, stream, D, token, args.steps, args.warmup, args.graph_steps, use_graph,
                               args.kernel_reps, weight_bits=4)

    line = {
        "metric": "decode tok/s (Gemma-2B shape, ctx 4K)",
        "value": round(tokens_per_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random N(0,0.02) bf16 weights, N(0,1) KV prefix, uniform prompt token; seed 0)",
        "config": {"workload": "gemma2-2b-shape greedy decode, batch 1, ctx 4096 -> 4096+steps (BASELINE config 4)",
                   "layers": cfg.layers, "hidden": cfg.hidden, "heads": f"{cfg.query_heads}q/{cfg.kv_heads}kv x {cfg.head_dim}",
                   "ffn": cfg.ffn, "vocab": cfg.vocab, "graph_steps": cfg.graph_steps if use_graph else 0,
                   "dispatches_per_step": nd},
        "hbm_step_GB_s": round(step_bytes * tokens_per_s / 1e9, 1),
        "hbm_step_frac": round(step_bytes * tokens_per_s / 1e9 / HBM_PEAK_GBS, 3),
        "roofline": roofline,
        "kernels": kernels,
        "in_step_sum_us": round(in_step_sum_us, 1),
        "flash_decoding_config2": fd,
        "mlp_config3": mlp,
        "prefill_config5": prefill,
        "decode_attention_block": block,
        "skinny_gemm": skinny,
        "q4_matvec": q4,
        "q4_prompt_gemm": q4p,
        "decode_q4": q4dec,
        "cpu_baseline": cpu,
    }
    dec.close()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
