"""Benchmark of the gfx950 LightOnOCR decode path on one MI355X.

Headline (value): greedy decode tokens/s at batch 1 of the random-init Qwen3-0.6B-shaped q8_0 decoder (28 layers, dim
1024, 16 / 8 heads × 128, SwiGLU 3072, vocab 151936, tied head): a 1024-token seeded prompt is prefilled once; one
step = one read of 512 greedy tokens with the windowed repetition penalty (64 / 1.1), chosen on the GPU, replayed as
HIP graphs. Each step rewinds the session to 1023 positions, runs one decode step for the prompt's last token and
decodes 512 tokens (so every step is the same read).

Also measured in the same run (one JSON line):
  roofline      the decode's own kernel, k_decode_token (one token in one launch): its algorithmic bytes per token at
                the read's mean context (1279.5 keys: 781,569,024 B) over its average launch time there (a graph of 16
                launches at 1280 keys, replayed; HIP events on the library's stream), against 8 TB/s; traffic from the
                committed FETCH_SIZE / WRITE_SIZE summary of the same kernel over the bench's read
  roofline_by_config
                every workload's fraction of its roofline: the decode (bytes per token × tokens/s), one matvec per
                graph node over the rotation and the q8_0 matvec kernel's streaming rate (k_dmv_many: 128 matvecs of
                W [3072 × 1024] per launch over 128 distinct copies, 430 MB > the 256 MB Infinity Cache), the choice
                per step (graphed) and 512 rows batched, the attention at 512 / 2048 / 8192 keys (graphed over
                ≥ 512 MiB of caches), the vision GEMMs (MFMA)
  decode.phases the decode step's kernel classes timed alone in graphs (htr_session_profile_step) at the read's mean
                context
  matvec        the same kernel one matvec per launch / per graph node over the rotation (and the 64-copy figure)
  choose        windowed penalty + argmax over 151936 logits: 10k seeded steps over 512 rows of the choice workload
                (planted maxima, 25 % repeated window ids), launched one by one and replayed as graphs, the rows
                restored between passes (each step sees its seeded logits); all rows batched; every pass's 512 tokens
                the same
  attention     GQA decode attention (16 q / 8 kv heads × 128) at 512 / 2048 / 8192 keys over ≥ 512 MiB of rotating caches
  copy, read    a 512 MiB device copy (the byte counters' reference point) and a read of the matvec's 430 MB and
                nothing else (the read rate a streaming kernel can reach: htr_debug_read)
  handover      the one-launch step's hand-over on its own (htr_debug_handover)
  vision_gemm, vision_encode
                a vision layer's GEMMs at 12100 rows against the dense f16 MFMA peak; a 1540 × 1540 page end to end
  cpu_baseline  the oracle (oracle/, a C restatement of the reference path, OpenMP) decoding the read's own keys 1024 …
                1535 on the host cores from the GPU's prefill rows, and the choice on the choose leg's 512 rows, whose
                tokens it checks
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "historic-htr-ocr_amd"))

import htr  # noqa: E402

HBM_PEAK_GBS = 8000.0
MATVEC_UNIT_BYTES = 3072 * 1024 + 3072 * 32 * 2 + 1024 * 4 + 3072 * 4  # W quants + scales + x + y = 3,358,720
CHOOSE_STEP_BYTES = 151936 * 4 + 64 * 4  # the logits read once + the window's ids
# one decode token of the 28-layer model at n_keys keys: the q8_0 weights (quants + scales, the tied LM head included),
# the norm weights, the K / V rows of every layer read and the new one written, the logits written and read back
DECODE_WEIGHT_BYTES = 633_233_408
DECODE_NORM_BYTES = 262_144
KV_BYTES_PER_KEY = 28 * 2 * 8 * 128 * 2  # 114,688
LOGIT_BYTES = 2 * 151936 * 4


def decode_bytes_per_token(mean_keys: float) -> float:
    return DECODE_WEIGHT_BYTES + DECODE_NORM_BYTES + KV_BYTES_PER_KEY * (mean_keys + 1) + LOGIT_BYTES


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def prefill_on_f32_path(dev, cfg, te, on, layers, ids) -> float:
    """the same prefill on the F32 compute path (exact q8_0 values in the GEMMs): a second model, a warm call timed"""
    keep = dev.compute
    dev.compute = htr.COMPUTE_F32
    try:
        m = htr.TextModel(dev, htr.TextConfig(**cfg), te, on, layers)
    finally:
        dev.compute = keep
    s = m.session(len(ids))
    s.prefill(ids)
    s.rewind(0)
    dev.sync()
    t0 = time.perf_counter()
    s.prefill(ids)
    dt = time.perf_counter() - t0
    log(f"prefill {len(ids)} tokens (f32 path): {dt * 1e3:.1f} ms")
    s.free()
    m.free()
    return dt


def bench_decode(dev, steps: int, warmup: int, prompt_len=1024, n_new=512, ab=True, n_ctx=None):
    from htr import synth

    t = time.time()
    cfg, te, on, layers = synth.text_model()
    log(f"decoder weights generated ({time.time() - t:.1f} s)")
    m = htr.TextModel(dev, htr.TextConfig(**cfg), te, on, layers)
    log("decoder weights uploaded")
    prompt = synth.prompt_ids(4242, prompt_len, cfg["n_vocab"])
    s = m.session(n_ctx or prompt_len + n_new)
    dev.sync()
    t0 = time.perf_counter()
    s.prefill(prompt[:-1])
    prefill_cold_s = time.perf_counter() - t0
    # the first call also loads the kernels' code objects and sizes the session's row buffers;
    # the warm figure re-runs the same prompt from position 0
    s.rewind(0)
    dev.sync()
    t0 = time.perf_counter()
    s.prefill(prompt[:-1])
    prefill_s = time.perf_counter() - t0
    path = "f16" if dev.compute == htr.COMPUTE_F16 else "f32"
    log(f"prefill {prompt_len - 1} tokens ({path} path): {prefill_s * 1e3:.1f} ms (first call {prefill_cold_s * 1e3:.1f} ms)")
    preset = htr.Preset(repetition_penalty=1.1, repetition_window=64, max_new_tokens=n_new)
    ch = s.choice(preset, prompt, chunk=16, depth=2)
    fused = s.fused_step
    form = "one launch a token (embed, 28 layers, LM head, choice)" if fused else "per kernel"

    def reads_of(sess, chc, n_reads, n_warm):
        def one_read():
            sess.rewind(prompt_len - 1)
            sess.step(int(prompt[-1]))
            return sess.decode_gpu(chc, n_new)

        ref = None
        for i in range(n_warm):
            toks = one_read()
            ref = ref or toks
        dev.sync()
        t0 = time.perf_counter()
        got = [one_read() for _ in range(n_reads)]
        dev.sync()
        return got, time.perf_counter() - t0, ref

    reads, dt, ref = reads_of(s, ch, steps, warmup)
    same = all(r == reads[0] for r in reads) and (ref is None or ref == reads[0])
    log(f"decode ({form}): {steps} reads × {n_new} tokens in {dt:.3f} s, identical reads: {same}")
    # the read's steps run at 1024 … 1535 keys (mean 1279.5)
    mean_keys = (prompt_len + prompt_len + n_new - 1) / 2
    bpt = decode_bytes_per_token(mean_keys)
    tok_s = steps * n_new / dt
    mid = prompt_len - 1 + n_new // 2
    fused_phases = fused_step_phases(s, mid, int(prompt[5]), cfg["n_layer"]) if fused else None
    instance = dev.last_kernel()  # the one-launch step's instance (the A/B legs below launch other kernels)
    # the same read on the per-kernel step (A/B in one run), and its kernel classes in graphs
    per_kernel, phases = None, None
    if fused and ab:
        sk = m.session(n_ctx or prompt_len + n_new)
        sk.fused_step = False
        sk.prefill(prompt[:-1])
        chk = sk.choice(preset, prompt, chunk=16, depth=2)
        rk, dtk, _ = reads_of(sk, chk, max(1, steps // 2), 1)
        per_kernel = {"tok_s": len(rk) * n_new / dtk, "ms_per_token": dtk / (len(rk) * n_new) * 1e3,
                      "same_tokens": rk[0] == reads[0]}
        log(f"decode (per kernel): {per_kernel['tok_s']:.1f} tok/s, the same tokens: {per_kernel['same_tokens']}")
        phases = decode_phases(sk, mid, cfg["n_layer"]) if GRAPHS else None
        chk.free()
        sk.free()
    elif ab:
        phases = decode_phases(s, mid, cfg["n_layer"]) if GRAPHS else None
    prefill_f32_s = (prefill_on_f32_path(dev, cfg, te, on, layers, prompt[:-1]) if path == "f16" else prefill_s) \
        if ab else float("nan")
    # the one-launch step's average launch at the read's mean context: a graph of 16 launches at position 1279
    # (1280 keys), replayed, HIP events on the library's stream (htr_session_profile_step)
    kernel_us = fused_phases["step_in_graph_us"] if fused_phases else float("nan")
    out = {
        "step_form": form,
        "kernel_us_at_mean_keys": kernel_us,
        "kernel_instance": instance,
        "tok_s": tok_s,
        "bytes_per_token": bpt,
        "mean_keys": mean_keys,
        "achieved_GBs": bpt * tok_s / 1e9,
        "frac": bpt * tok_s / 1e9 / HBM_PEAK_GBS,
        "roofline_tok_s": HBM_PEAK_GBS * 1e9 / bpt,
        "fused_step_phases": fused_phases,
        "per_kernel_step": per_kernel,
        "phases": phases,
        "ms_per_read": dt / steps * 1e3,
        "ms_per_token": dt / (steps * n_new) * 1e3,
        "prefill_ms": prefill_s * 1e3,
        "prefill_first_call_ms": prefill_cold_s * 1e3,
        "prefill_compute_path": path,
        "prefill_f32_path_ms": prefill_f32_s * 1e3,
        "reads_identical": same,
        "first_tokens": reads[0][:8],
        "first_tokens_all": reads[0],
    }
    return out, (cfg, te, on, layers, prompt), (m, s, ch)


def decode_phases(s, pos, n_layer, n_steps=16, reps=20):
    """the decode step's kernel classes each alone in a graph of n_steps steps at position pos (the read's mean
    context), and all of them together: µs per step and per layer"""
    s.rewind(pos)
    classes = [("embed", htr.STEP_EMBED), ("qkv_matvec", htr.STEP_QKV), ("attention", htr.STEP_ATTENTION),
               ("o_matvec", htr.STEP_O), ("gate_up_matvec", htr.STEP_FFN), ("down_matvec", htr.STEP_DOWN),
               ("lm_head", htr.STEP_HEAD), ("step", htr.STEP_ALL)]
    out = {"position": pos, "keys": pos + 1, "steps_per_graph": n_steps}
    for name, c in classes:
        us = s.profile_step(c, n_steps, reps) * 1e3
        per_layer = c not in (htr.STEP_EMBED, htr.STEP_HEAD, htr.STEP_ALL)
        out[name + "_us"] = us
        if per_layer:
            out[name + "_us_per_layer"] = us / n_layer
    out["sum_of_classes_us"] = sum(out[n + "_us"] for n, c in classes if c != htr.STEP_ALL)
    log("decode phases (µs a step, in graphs): " + ", ".join(f"{n} {out[n + '_us']:.1f}" for n, _ in classes))
    return out


def fused_step_phases(s, pos, tok, n_layer):
    """the one-launch step at position pos, timed from inside by workgroup 0's wall-clock stamps: per phase (qkv,
    attention, merge, o, gate/up, down) the wait for its input (from the previous phase's output written) and its own
    work (to its output written), µs averaged over the layers; and the step as a graph alone (profile_step)"""
    s.rewind(pos)
    us = s.profile_fused_step(tok)
    d = np.diff(us[: 1 + 12 * n_layer]).reshape(n_layer, 12)
    names = ["qkv", "attention", "merge", "o", "gate_up", "down"]
    out = {"position": pos, "keys": pos + 1, "kernel_us": float(us[-1])}
    for i, n in enumerate(names):
        out[n + "_wait_us"] = float(d[:, 2 * i].mean())
        out[n + "_work_us"] = float(d[:, 2 * i + 1].mean())
    out["layer_us"] = float(d.sum(1).mean())
    t = np.diff(us[12 * n_layer:])  # the LM head: its input's wait, its rows, the rest
    out["lm_head_wait_us"], out["lm_head_rows_us"], out["lm_head_tail_us"] = (float(x) for x in t)
    out["step_in_graph_us"] = s.profile_step(htr.STEP_ALL, 16, 20) * 1e3 if GRAPHS else float("nan")
    log("one-launch step (µs a layer): " + ", ".join(f"{n} wait {out[n + '_wait_us']:.2f} work {out[n + '_work_us']:.2f}"
                                                   for n in names)
        + f"; LM head wait {out['lm_head_wait_us']:.2f}, rows {out['lm_head_rows_us']:.2f}; kernel {out['kernel_us']:.1f} µs")
    return out


GRAPHS = True  # --no-graphs: the graph-recording legs are skipped (None in the line)


def graphed(dev, calls, reps):
    """µs per call of `calls` (a list of zero-argument functions, each one library entry point) recorded once into a
    graph and replayed reps times after one untimed replay"""
    if not GRAPHS:
        return float("nan")
    dev.capture_begin()
    try:
        for f in calls:
            f()
    finally:
        g = dev.capture_end()
    g.launch()
    dev.sync()
    dev.timer_begin()
    for _ in range(reps):
        g.launch()
    ms = dev.timer_end()
    g.free()
    return ms * 1e3 / (reps * len(calls))


def bench_matvec(dev, copies=128, reps=10):
    rows, k = 3072, 1024
    log(f"matvec: {copies} copies of W [{rows} x {k}]")
    ws = []
    base = htr.synth_q8_0(9000, rows, k)
    for i in range(copies):
        # distinct copies: every block's scale differs per copy (quants shared), so no two copies alias in any cache
        b = base.copy()
        b.reshape(-1, 34)[:, 0] ^= np.uint8(i & 0xFF)
        ws.append(htr.Weight(dev, b, rows, k))
    x = dev.upload(htr.synth_normal(9001, k))
    y = dev.alloc(copies * rows * 4)
    ys = dev.alloc(rows * 4)
    # one matvec per launch, rotating
    for w in ws[:8]:
        htr.matvec_q8_0(dev, w, x, ys)
    dev.sync()
    res = {}
    for n_rot in (copies, 64):
        dev.timer_begin()
        n_l = 0
        for _ in range(4):
            for w in ws[:n_rot]:
                htr.matvec_q8_0(dev, w, x, ys)
                n_l += 1
        ms = dev.timer_end()
        res[f"single_launch_{n_rot}_copies_us"] = ms / n_l * 1e3
        res[f"single_launch_{n_rot}_copies_GBs"] = MATVEC_UNIT_BYTES / (ms / n_l * 1e-3) / 1e9
        # one matvec per graph node (no host launch between them): the kernel's time with its node overhead
        us = graphed(dev, [lambda w=w: htr.matvec_q8_0(dev, w, x, ys) for w in ws[:n_rot]], 4)
        res[f"graph_node_{n_rot}_copies_us"] = us
        res[f"graph_node_{n_rot}_copies_GBs"] = MATVEC_UNIT_BYTES / (us * 1e-6) / 1e9
        res[f"graph_node_{n_rot}_copies_frac"] = res[f"graph_node_{n_rot}_copies_GBs"] / HBM_PEAK_GBS
    # all copies in one launch
    htr.matvec_q8_0_many(dev, ws, x, y)
    dev.timer_begin()
    for _ in range(reps):
        htr.matvec_q8_0_many(dev, ws, x, y)
    ms = dev.timer_end() / reps
    bytes_launch = copies * MATVEC_UNIT_BYTES
    res["batched_launch_us"] = ms * 1e3
    res["batched_launch_GBs"] = bytes_launch / (ms * 1e-3) / 1e9
    res["batched_bytes_per_launch"] = bytes_launch
    for w in ws:
        w.free()
    res["batched_frac"] = res["batched_launch_GBs"] / HBM_PEAK_GBS
    log(f"matvec: batched {res['batched_launch_GBs']:.0f} GB/s, single {res[f'single_launch_{copies}_copies_GBs']:.0f} "
        f"GB/s launched, {res[f'graph_node_{copies}_copies_GBs']:.0f} GB/s as graph nodes "
        f"({res[f'graph_node_{copies}_copies_us']:.2f} us)")
    return res


def bench_choose(dev, n_steps=10000, n_buf=512, n_vocab=151936, window=64):
    """the choice workload (htr.synth.choice_inputs: N(0, 3) logits with 8 planted equal maxima, 3 on window ids; 64
    uniform window ids with 25 % repeats) in 512 rows, 311 MB of logits: 10k single steps over the rows launched one by
    one (passes of 512 steps), the same replayed as graphs of 512 steps, and all rows in one launch. The choice
    penalises its row in place, so the rows are restored from a pristine copy between passes (untimed): every step sees
    its row's seeded logits, an independent step. Each row's token has its own slot; every pass must give the same 512
    tokens (the CPU leg checks them against the oracle's choice on the same rows). → (result, (host logits, host
    windows, tokens))"""
    from htr import synth

    log(f"choose: {n_steps} steps over {n_buf} rows of the choice workload")
    logits = dev.alloc(n_buf * n_vocab * 4)
    pristine = dev.alloc(n_buf * n_vocab * 4)
    host_l = np.empty((n_buf, n_vocab), np.float32)
    hist_h = np.zeros((n_buf, window + 1), np.uint32)
    block = 32
    for i in range(0, n_buf, block):
        lg, h = synth.choice_inputs(7000 + i, block, n_vocab, window)
        host_l[i:i + block] = lg
        hist_h[i:i + block, :window] = h
    pristine.upload(host_l)
    hist = dev.upload(hist_h)
    tok = dev.alloc(n_buf * 4)
    L = htr.lib()
    stride = (window + 1) * 4

    def one(i):
        r = i % n_buf
        rc = L.htr_choose(dev.h, logits.ptr + r * n_vocab * 4, n_vocab, hist.ptr + r * stride, window, window, 1.1,
                          0.0, None, None, tok.ptr + 4 * r)
        if rc < 0:
            raise htr.HtrError(htr.last_error())

    def restore():
        logits.copy_from(pristine)
        dev.sync()

    restore()
    for i in range(16):
        one(i)
    restore()
    passes, ms, done = [], 0.0, 0
    while done < n_steps:
        n = min(n_buf, n_steps - done)
        dev.timer_begin()
        for i in range(n):
            one(i)
        ms += dev.timer_end()
        passes.append(tok.download(np.uint32, n).copy())
        restore()
        done += n
    n_rows = passes[0].size  # the rows of the first pass (all 512 unless fewer steps were asked)
    same = all(np.array_equal(p, passes[0][:p.size]) for p in passes)
    res = {"steps": n_steps, "us_per_step": ms / n_steps * 1e3, "GBs": CHOOSE_STEP_BYTES / (ms / n_steps * 1e-3) / 1e9,
           "passes_of_512": len(passes), "passes_identical": same,
           "rows_restored_between_passes": True}
    # graphs of 512 steps, replayed once per pass with the rows restored between replays
    if GRAPHS:
        dev.capture_begin()
        try:
            for i in range(n_buf):
                one(i)
        finally:
            g = dev.capture_end()
        g.launch()
        restore()
        reps = max(1, n_steps // n_buf)
        ms_g = 0.0
        for _ in range(reps):
            dev.timer_begin()
            g.launch()
            ms_g += dev.timer_end()
            same = same and np.array_equal(tok.download(np.uint32, n_rows), passes[0])
            restore()
        g.free()
        us = ms_g * 1e3 / (reps * n_buf)
        res["graph_passes_identical"] = same
    else:
        us = float("nan")
    res["graph_node_us_per_step"] = us
    res["graph_node_GBs"] = CHOOSE_STEP_BYTES / (us * 1e-6) / 1e9
    res["graph_node_frac"] = res["graph_node_GBs"] / HBM_PEAK_GBS
    # the 512 rows in one launch (independent rows, each with its own window), restored between launches
    toks = dev.alloc(n_buf * 4)
    htr.choose_many(dev, logits, n_vocab, n_buf, hist, window + 1, window, window, 1.1, toks)
    batched_kernel = dev.last_kernel()
    batched_same = np.array_equal(toks.download(np.uint32, n_rows), passes[0])
    restore()
    ms = 0.0
    for _ in range(5):
        dev.timer_begin()
        htr.choose_many(dev, logits, n_vocab, n_buf, hist, window + 1, window, window, 1.1, toks)
        ms += dev.timer_end()
        restore()
    ms /= 5
    res["batched_rows_per_launch"] = n_buf
    res["batched_kernel"] = batched_kernel
    res["batched_tokens_equal_single_steps"] = batched_same
    res["batched_us_per_row"] = ms / n_buf * 1e3
    res["batched_GBs"] = n_buf * CHOOSE_STEP_BYTES / (ms * 1e-3) / 1e9
    res["batched_frac"] = res["batched_GBs"] / HBM_PEAK_GBS
    for b in (logits, pristine, hist, tok, toks):
        b.free()
    log(f"choose: {res['us_per_step']:.2f} us/step launched, {us:.2f} us as graph nodes, batched "
        f"{res['batched_GBs']:.0f} GB/s; every pass the same 512 tokens: {same}")
    return res, (host_l[:n_rows], hist_h[:n_rows, :window].astype(np.int64), passes[0].astype(np.int64))


def bench_attention(dev, n_head=16, n_kv=8, rotate_mib=512):
    """GQA decode attention at 512 / 2048 / 8192 keys, each call on another copy of the caches (≥ 512 MiB of them, past
    the 256 MB Infinity Cache): launched one by one and replayed as graphs"""
    res = {}
    q = dev.upload(htr.synth_normal(31, n_head * 128))
    out = dev.alloc(n_head * 128 * 4)
    L_ = htr.lib()
    sc = float(np.float32(1 / np.sqrt(128)))
    for L in (512, 2048, 8192):
        per = 2 * n_kv * L * 128 * 2
        copies = max(8, -(-rotate_mib * 2 ** 20 // per))
        kv = dev.alloc(copies * per)
        a = htr.synth_normal(L, 2 * n_kv * L * 128).astype(np.float16)
        for c in range(copies):
            L_.htr_upload(dev.h, kv.ptr + c * per, a.ctypes.data, a.nbytes)
        half = per // 2

        def one(c, L=L, kv=kv, per=per, half=half):
            rc = L_.htr_decode_attention(dev.h, q.ptr, kv.ptr + c * per, kv.ptr + c * per + half, n_head, n_kv, L, L,
                                         sc, out.ptr)
            if rc < 0:
                raise htr.HtrError(htr.last_error())

        for c in range(4):
            one(c)
        n = 4 * copies
        dev.timer_begin()
        for i in range(n):
            one(i % copies)
        ms = dev.timer_end() / n
        byts = 4096 * L + 16384
        us_g = graphed(dev, [lambda c=c: one(c) for c in range(copies)], max(1, 512 // copies))
        res[str(L)] = {"us": ms * 1e3, "GBs": byts / (ms * 1e-3) / 1e9, "copies": copies,
                       "rotation_MiB": copies * per / 2 ** 20, "graph_node_us": us_g,
                       "graph_node_GBs": byts / (us_g * 1e-6) / 1e9,
                       "graph_node_frac": byts / (us_g * 1e-6) / 1e9 / HBM_PEAK_GBS}
        kv.free()
        log(f"attention L={L}: {ms * 1e3:.2f} us launched, {us_g:.2f} us as graph nodes, "
            f"{res[str(L)]['graph_node_GBs']:.0f} GB/s")
    return res


MFMA_F16_PEAK_TFLOPS = 2500.0


def bench_vision_gemm(dev, reps=5, m=12100, dim=1024, ff=4096):
    """the vision encoder layer's GEMMs on the matrix cores at one page's 12100 patch rows, as the encoder runs them:
    Q / K / V as one GEMM over the stacked [3072 x 1024] weights, o [1024 x 1024] onto the residual, gate + up
    [4096 x 1024] x 2 fused with SwiGLU, down [1024 x 4096] onto the residual (q8_0 weights dequantised to f16 at
    load)"""
    x16 = dev.upload(synth_normal_f16(71, m * ff))
    y = dev.alloc(m * 3 * dim * 4)
    g16 = dev.alloc(m * ff * 2)
    ws = {name: htr.Weight(dev, htr.synth_q8_0(600 + i, rows, cols), rows, cols, f16=True,
                           scale=64.0 if name == "down" else 1.0)
          for i, (name, rows, cols) in enumerate([("qkv", 3 * dim, dim), ("o", dim, dim), ("gate", ff, dim),
                                                  ("up", ff, dim), ("down", dim, ff)])}

    def layer():
        htr.gemm_f16(dev, x16, m, ws["qkv"], y)
        htr.gemm_f16(dev, x16, m, ws["o"], y, acc=True)
        htr.gemm_ffn_f16(dev, x16, m, ws["gate"], ws["up"], 1.0 / 64, g16)
        htr.gemm_f16(dev, g16, m, ws["down"], y, acc=True)

    layer()
    dev.timer_begin()
    for _ in range(reps):
        layer()
    ms = dev.timer_end() / reps
    flop = 2.0 * m * (4 * dim * dim + 2 * ff * dim + dim * ff)
    # the single largest GEMM alone (gate + up, 2 x 101.5 GFLOP)
    dev.timer_begin()
    for _ in range(reps):
        htr.gemm_ffn_f16(dev, x16, m, ws["gate"], ws["up"], 1.0 / 64, g16)
    ms_ffn = dev.timer_end() / reps
    for w in ws.values():
        w.free()
    res = {"rows": m, "layer_gemm_ms": ms, "layer_gemm_flop": flop, "tflops": flop / (ms * 1e-3) / 1e12,
           "ffn_ms": ms_ffn, "ffn_tflops": 2.0 * m * 2 * ff * dim / (ms_ffn * 1e-3) / 1e12}
    res["frac_mfma_peak"] = res["tflops"] / MFMA_F16_PEAK_TFLOPS
    res["encoder_gemm_ms_24_layers"] = 24 * ms
    log(f"vision GEMMs: {ms:.3f} ms per layer ({res['tflops']:.0f} TFLOP/s, {100 * res['frac_mfma_peak']:.1f} % of "
        f"the f16 MFMA peak); FFN gate/up {res['ffn_tflops']:.0f} TFLOP/s")
    return res


def bench_vision_encode(dev, reps=5):
    """the vision encoder end to end: one 1540 x 1540 page (12100 patches) through the 24-layer encoder and the projector
    (3025 x 1024 embeddings left on the device), random-init q8_0 weights"""
    from htr import synth

    cfg, t = synth.vision_model()
    v = htr.Vision(dev, cfg, t)
    rgb = synth.page(99, 1540, 1540)
    out, n, d = v.encode_gpu(rgb)
    dev.timer_begin()
    for _ in range(reps):
        v.encode_gpu(rgb, out=out)
    ms = dev.timer_end() / reps
    emb = out.download(np.float32, n * d)
    out.free()
    v.free()
    m = 12100
    gemm = 24 * 2.0 * m * (4 * 1024 * 1024 + 3 * 4096 * 1024)
    attn = 24 * 16 * 2 * (2.0 * m * m * 64)
    res = {"page": "1540x1540", "patches": m, "out_tokens": n, "encode_ms": ms, "gemm_flop": gemm,
           "attention_flop": attn, "finite": bool(np.all(np.isfinite(emb)))}
    log(f"vision encode 1540x1540: {ms:.1f} ms per page ({n} x {d} embeddings)")
    return res


def synth_normal_f16(seed, n):
    return htr.synth_normal(seed, n).astype(np.float16)


def bench_copy(dev, mib=512, reps=5):
    """a plain device copy of known size (htr_copy): the HBM reference point of the byte counters"""
    n = mib << 20
    src, dst = dev.alloc(n), dev.alloc(n)
    dst.copy_from(src)
    dev.timer_begin()
    for _ in range(reps):
        dst.copy_from(src)
    ms = dev.timer_end() / reps
    src.free()
    dst.free()
    res = {"bytes": n, "us": ms * 1e3, "GBs_read_plus_write": 2 * n / (ms * 1e-3) / 1e9}
    log(f"copy {mib} MiB: {res['us']:.1f} us, {res['GBs_read_plus_write']:.0f} GB/s (read + write)")
    return res


def bench_read(dev, nbytes=429916160, reps=20):
    """a read of known size and nothing else (htr_debug_read): the read rate a streaming kernel can reach on this
    device, over the batched matvec's own byte count (128 W copies, past the 256 MB Infinity Cache); 16 / 32 / 64 KB a
    workgroup, plain and non-temporal 16-byte loads"""
    buf, sink = dev.alloc(nbytes), dev.alloc(4)
    res = {"bytes": nbytes}
    for nt in (True, False):
        for kb in (16, 32, 64):
            buf.read_through(sink, nt, kb)
            dev.timer_begin()
            for _ in range(reps):
                buf.read_through(sink, nt, kb)
            us = dev.timer_end() / reps * 1e3
            res[f"{'nontemporal' if nt else 'plain'}_{kb}KB_a_workgroup_GBs"] = nbytes / (us * 1e-6) / 1e9
    buf.free()
    sink.free()
    res["best_GBs"] = max(v for k, v in res.items() if k.endswith("_GBs"))
    res["best_frac_of_peak"] = res["best_GBs"] / HBM_PEAK_GBS
    log("read " + ", ".join(f"{k[:-4]} {v:.0f}" for k, v in res.items() if k.endswith("workgroup_GBs"))
        + f" GB/s; best {res['best_GBs']:.0f} GB/s ({res['best_frac_of_peak']:.3f} of 8 TB/s)")
    return res


def bench_handover(dev):
    """the hand-over the one-launch decode step rests on (htr_debug_handover, 256 workgroups of one launch): one tagged
    word back and forth between two workgroups on one XCD (0 and 8) and on two (0 and 1), stored at workgroup scope
    (kept in the writer XCD's L2) or agent scope (written through), read with agent-scope loads; and all-to-all
    exchanges of 1024 / 2048 / 3072 words with the first poll 16 × 64 clocks after a workgroup's own words (1024 words
    also at 0, 8, 12 and 24)"""
    res = {}
    for kind, scope in ((0, "workgroup"), (1, "agent")):
        for a, b, where in ((0, 8, "one_xcd"), (0, 1, "two_xcds")):
            # a workgroup-scope word is not seen from another XCD: a short limit ends that wait
            us, seen = dev.handover(kind, a, b, iters=2000, max_polls=(1 << 20) if kind or where == "one_xcd" else 4096)
            res[f"pair_{scope}_store_{where}"] = {"round_trip_us": us if seen else None, "seen": seen}
    for words, pause in ((1024, 16), (2048, 16), (3072, 16), (1024, 0), (1024, 8), (1024, 12), (1024, 24)):
        us, seen = dev.handover(2, words=words, pause=pause, iters=1000)
        res[f"all_to_all_{words}_words_pause_{pause}"] = {"exchange_us": us if seen else None, "seen": seen}
    f = lambda v: "not seen" if v is None else f"{v:.3f}"
    log("hand-over (µs): one word's round trip, stored at workgroup scope: one XCD "
        f"{f(res['pair_workgroup_store_one_xcd']['round_trip_us'])}, two XCDs "
        f"{f(res['pair_workgroup_store_two_xcds']['round_trip_us'])}; at agent scope: one XCD "
        f"{f(res['pair_agent_store_one_xcd']['round_trip_us'])}, two XCDs {f(res['pair_agent_store_two_xcds']['round_trip_us'])}"
        "; an all-to-all exchange: " + ", ".join(f"{k[11:]} {f(v['exchange_us'])}" for k, v in res.items()
                                                if k.startswith("all_to_all")))
    return res


def load_traffic(name="k_dmv_many_w3072x1024_traffic.json", key="hbm_bytes_per_launch"):
    """HBM bytes per launch of the roofline kernel (or per token of the decode kernel) from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by what the same counters read for a copy of known
    size), or None"""
    f = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(f):
        return None
    with open(f) as fh:
        t = json.load(fh)
    if key == "hbm_bytes_per_token":
        return t["hbm_fetch_bytes_per_token"] + t["hbm_write_bytes_per_token"] if "hbm_fetch_bytes_per_token" in t else None
    return t.get(key)


def _timed(fn, budget_s, min_n=3):
    """(calls, seconds) of fn() repeated until budget_s has passed (at least min_n calls)"""
    n, t0 = 0, time.perf_counter()
    while n < min_n or time.perf_counter() - t0 < budget_s:
        fn()
        n += 1
    return n, time.perf_counter() - t0


def cpu_configs(orc, threads, choice_rows=None, budget_s=2.0):
    """the oracle on the host cores for the other single-kernel workloads: the q8_0 matvec W [3072 x 1024], the
    penalised greedy choice over 151,936 logits (window 64, rp 1.1) — on the choose leg's own 512 rows, whose tokens it
    checks — and the decode attention (16 / 8 heads x 128) at 512 / 2048 / 8192 keys"""
    r = np.random.default_rng(0)
    w = orc.q8_0_quantize(r.normal(0, 1, 3072 * 1024).astype(np.float32))[0]
    x = r.normal(0, 1, 1024).astype(np.float32)
    n, dt = _timed(lambda: orc.matvec_q8_0(w, 3072, 1024, x), budget_s)
    res = {"matvec_w3072x1024": {"us": dt / n * 1e6, "GBs": MATVEC_UNIT_BYTES / (dt / n) / 1e9, "calls": n}}
    if choice_rows is not None:
        host_l, hist, gpu_toks = choice_rows
        spent, agree = 0.0, 0
        for i in range(host_l.shape[0]):
            lo = host_l[i].copy()  # choose penalises in place: a fresh row each step, copied outside the timing
            t0 = time.perf_counter()
            t = orc.choose(lo, 1.1, 64, 0.0, [int(v) for v in hist[i]])
            spent += time.perf_counter() - t0
            agree += int(t == gpu_toks[i])
        res["choose_151936"] = {"us": spent / host_l.shape[0] * 1e6, "calls": host_l.shape[0],
                                "rows_checked": host_l.shape[0], "gpu_tokens_equal": agree == host_l.shape[0],
                                "gpu_tokens_equal_count": agree}
    q = r.normal(0, 1, 16 * 128).astype(np.float32)
    sc = float(np.float32(1 / np.sqrt(128)))
    for L in (512, 2048, 8192):
        kv = r.normal(0, 1, (2, L, 8, 128)).astype(np.float16).view(np.uint16)  # the oracle's [key][kv head][128]
        n, dt = _timed(lambda: orc.attn_decode(q, kv[0], kv[1], 8 * 128, L, 16, 8, sc), budget_s / 3)
        res[f"attention_{L}"] = {"us": dt / n * 1e6, "GBs": (4096 * L + 16384) / (dt / n) / 1e9, "calls": n}
    res["threads"] = threads
    return res


def cpu_baseline(model_inputs, prefill_rows, choice_rows=None, budget_s=25.0, n_new=512):
    """the oracle (C restatement of the reference decode path, OpenMP) decoding the workload on the host cores: the
    GPU's prefill rows 0 … 1022 of every layer handed to it, one step for the prompt's last token, then greedy tokens
    (rp 1.1 / 64) over keys 1024 … 1535 — the measured read's own keys — until the read's 512 or the time budget; the
    other single-kernel workloads timed the same way under per_config"""
    # the oracle (test infrastructure): imported here, for the CPU baseline leg only
    import importlib.util

    spec = importlib.util.spec_from_file_location("htr_oracle_py", os.path.join(ROOT, "oracle", "oracle.py"))
    orc = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(orc)

    cfg, te, on, layers, prompt = model_inputs
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    n0 = len(prompt) - 1
    o = orc.Session(cfg, te, on, layers, len(prompt) + n_new, f16=True)  # the measured path's fused step
    for li, (k, v) in enumerate(prefill_rows):
        o.set_kv(li, 0, k, v)
    o.rewind(n0)
    lo = o.step(int(prompt[-1]))
    hist = [int(t) for t in prompt]
    toks = []
    t0 = time.perf_counter()
    n = 0
    while n < n_new and (n < 3 or time.perf_counter() - t0 < budget_s):
        t = orc.choose(lo, 1.1, 64, 0.0, hist)
        hist.append(t)
        toks.append(t)
        n += 1
        if n < n_new:
            lo = o.step(t)
    dt = time.perf_counter() - t0
    log(f"cpu baseline: {n} tokens in {dt:.1f} s on {threads} threads (keys {n0 + 1} … {n0 + n})")
    per = cpu_configs(orc, threads, choice_rows)
    ch = per.get("choose_151936", {})
    log(f"cpu baseline: matvec {per['matvec_w3072x1024']['GBs']:.1f} GB/s, choose {ch.get('us', float('nan')):.0f} us "
        f"(the GPU's 512 tokens of the choose leg equal: {ch.get('gpu_tokens_equal')}), attention 8192 keys "
        f"{per['attention_8192']['us']:.0f} us")
    return {"value": n / dt, "unit": "tokens/s", "cores": threads, "kind": "port", "per_config": per,
            "tokens": toks,
            "sample": f"oracle (C restatement, OpenMP; the f16 paths' fused step) greedy decode of {n} tokens (rp 1.1 / "
                      f"64) of the same 28-layer q8_0 model from the GPU's prefill rows of the same 1024-token prompt: "
                      f"keys {n0 + 1}-{n0 + n}, the measured read's own"}


def no_nan(v):
    """NaN (a leg skipped with --no-graphs) and ±inf → null, so that the line is strict JSON"""
    if isinstance(v, float) and (v != v or v in (float("inf"), float("-inf"))):
        return None
    if isinstance(v, dict):
        return {k: no_nan(x) for k, x in v.items()}
    if isinstance(v, list):
        return [no_nan(x) for x in v]
    return v


def roofline_by_config(r: dict) -> dict:
    """each workload's achieved rate as a fraction of the bound that caps it (HBM 8 TB/s; the vision GEMMs: dense f16
    MFMA 2.5 PFLOP/s)"""
    out = {}
    if "decode" in r:
        d = r["decode"]
        out["config3_decode"] = {"bound": "hbm", "achieved_GBs": d["achieved_GBs"], "frac": d["frac"],
                                 "unit": f"{d['bytes_per_token']:.0f} B a token at {d['mean_keys']} keys on average",
                                 "traffic_bytes_per_token": load_traffic("k_decode_token_traffic.json",
                                                                         "hbm_bytes_per_token")}
    if "matvec" in r:
        m = r["matvec"]
        out["config0_matvec_graph_node"] = {"bound": "hbm", "achieved_GBs": m["graph_node_128_copies_GBs"],
                                            "frac": m["graph_node_128_copies_frac"],
                                            "unit": "one W [3072 x 1024] matvec a graph node, 128 copies rotated"}
        out["config0_matvec_batched"] = {"bound": "hbm", "achieved_GBs": m["batched_launch_GBs"],
                                         "frac": m["batched_frac"], "kernel": "k_dmv_many",
                                         "avg_launch_us": m["batched_launch_us"],
                                         "algorithmic_bytes_per_launch": m["batched_bytes_per_launch"],
                                         "traffic": load_traffic(),
                                         "unit": "128 matvecs in one launch over 128 distinct W copies (430 MB, past "
                                                 "the 256 MB Infinity Cache): the kernel's streaming rate"}
        if "read" in r:
            out["config0_matvec_batched"]["frac_of_read_ceiling"] = m["batched_launch_GBs"] / r["read"]["best_GBs"]
    if "choose" in r:
        c = r["choose"]
        out["config1_choice_graph_node"] = {"bound": "hbm", "achieved_GBs": c["graph_node_GBs"],
                                            "frac": c["graph_node_frac"], "unit": "one step a graph node"}
        out["config1_choice_batched"] = {"bound": "hbm", "achieved_GBs": c["batched_GBs"], "frac": c["batched_frac"],
                                         "kernel": c.get("batched_kernel"), "unit": "512 steps in one launch"}
    if "attention" in r:
        for L, a in r["attention"].items():
            out[f"config2_attention_{L}"] = {"bound": "hbm", "achieved_GBs": a["graph_node_GBs"],
                                             "frac": a["graph_node_frac"], "unit": "one call a graph node"}
    if "vision_gemm" in r:
        v = r["vision_gemm"]
        out["config4_vision_gemm"] = {"bound": "mfma", "achieved_TFLOPs": v["tflops"], "frac": v["frac_mfma_peak"],
                                      "unit": "a layer's six GEMMs at 12100 rows"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--prompt", type=int, default=1024,
                    help="the decode leg's prompt length (the workload: 1024; longer ones measure longer contexts)")
    ap.add_argument("--ctx", type=int, default=0, help="the decode leg's session rows (default: prompt + 512)")
    ap.add_argument("--only", default="", help="comma list of: decode, matvec, choose, attention, copy (and the read leg), handover, vision")
    ap.add_argument("--choose-steps", type=int, default=10000,
                    help="single-launch steps of the choose leg (a counter run takes fewer: every launch is sampled)")
    ap.add_argument("--no-graphs", action="store_true",
                    help="skip the legs that record graphs (decode phases, graph-node timings): for profilers that "
                         "cannot follow stream capture (with HTR_GRAPHS=0 the decode launches its kernels one by one)")
    ap.add_argument("--no-ab", action="store_true",
                    help="the decode leg's one-launch read alone: no per-kernel A/B read, no kernel-class timing, no "
                         "F32-path prefill (counter runs of the decode kernel)")
    args = ap.parse_args()
    global GRAPHS
    GRAPHS = not args.no_graphs
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this path has no multi-GPU sharding (asked for {args.gpus})", file=sys.stderr)
        sys.exit(2)
    only = set(filter(None, args.only.split(",")))
    want = lambda k: not only or k in only
    dev = htr.Device(0)
    name, n_cu = dev.info()
    log(f"device {name}, {n_cu} CUs")
    result = {
        "metric": "decode tokens/sec at batch 1; q8_0 matvec HBM GB/s (% of peak)",
        "value": None,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded random-init q8_0 weights and prompt ids",
        "config": {"workload": "greedy decode at batch 1: 28-layer Qwen3-0.6B-shaped q8_0 decoder (dim 1024, 16/8 "
                               "heads x 128, SwiGLU 3072, vocab 151936, tied head), 1024-token prompt, 512 tokens, "
                               "repetition penalty 1.1 over a 64-token window; one step = one 512-token read",
                   "device": name},
    }
    decode_inputs, prefill_rows, choice_rows = None, None, None
    dev.phase("decode")
    if want("decode"):
        d, decode_inputs, keep = bench_decode(dev, args.steps, args.warmup, prompt_len=args.prompt, ab=not args.no_ab,
                                              n_ctx=args.ctx or None)
        result["value"] = d["tok_s"]
        result["ms_per_step"] = d["ms_per_read"]
        result["decode"] = d
        kus = d["kernel_us_at_mean_keys"]
        if kus == kus:
            ach = d["bytes_per_token"] / (kus * 1e-6) / 1e9
            result["roofline"] = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": ach / HBM_PEAK_GBS,
                                  "traffic": load_traffic("k_decode_token_traffic.json", "hbm_bytes_per_token"),
                                  "kernel": f"{d['kernel_instance']}: one decode token of the 28-layer q8_0 decoder in "
                                            "one launch (embed, 28 layers, LM head, greedy choice)",
                                  "algorithmic_bytes_per_launch": d["bytes_per_token"],
                                  "avg_launch_us": kus,
                                  "launch_timing": f"a graph of 16 launches at {int(d['mean_keys'] + 0.5)} keys (the "
                                                   "read's mean), replayed 20 times, HIP events on the library's "
                                                   "stream"}
        if not args.skip_cpu:
            m_, s_, _ = keep
            prefill_rows = [s_.kv_rows(li, 0, len(decode_inputs[4]) - 1) for li in range(decode_inputs[0]["n_layer"])]
        for obj in keep[::-1]:
            obj.free()
    dev.phase("matvec")
    if want("matvec"):
        mv = bench_matvec(dev)
        result["matvec"] = mv
    dev.phase("choose")
    if want("choose"):
        result["choose"], choice_rows = bench_choose(dev, n_steps=args.choose_steps)
    dev.phase("attention")
    if want("attention"):
        result["attention"] = bench_attention(dev)
    dev.phase("copy")
    if want("copy"):
        result["copy"] = bench_copy(dev)
        result["read"] = bench_read(dev)
    dev.phase("handover")
    if want("handover"):
        result["handover"] = bench_handover(dev)
    dev.phase("vision")
    if want("vision"):
        result["vision_gemm"] = bench_vision_gemm(dev)
        result["vision_encode"] = bench_vision_encode(dev)
    dev.phase("-")
    result["roofline_by_config"] = roofline_by_config(result)
    if decode_inputs is not None and not args.skip_cpu:
        cb = cpu_baseline(decode_inputs, prefill_rows, choice_rows)
        toks = cb.pop("tokens")
        cb["same_tokens_as_gpu_read"] = toks == result["decode"]["first_tokens_all"][:len(toks)]
        result["cpu_baseline"] = cb
    if "decode" in result:
        result["decode"].pop("first_tokens_all")
    dev.close()
    print(json.dumps(no_nan(result)), flush=True)


if __name__ == "__main__":
    main()
