"""Benchmark of the MI355X Qwen3.5 GGUF decode hot path.

Workloads (synthetic, seeded random-init weights in the named GGUF codec):
  decode (default)  2B-shaped Q4_K hybrid model (hidden 2048, 24 layers at
         3:1 GDN:attention, FFN 6144, vocab 151936), continuous-batch greedy
         decode at B=1 and B=32, each row holding a 2048-token random prefix in
         the bf16 KV cache and a random GDN state.  A step is one decode
         position for every row: embedding, 24 layers, LM head, device argmax
         feeding the next step's tokens.  value = B=1 tokens/s.
  decode_q8  the same model and step with Q8_0 weights (the codec of the
         reference's pinned checkpoints) at B=1 and B=4; value = B=1 tokens/s.
  decode_mixed  as decode_q8 with the mixed-quant layout (Q6_K embedding and
         LM head, V and FFN down, Q4_1 attention gate, F32 GDN alpha/beta).
  gemv   dequant-GEMV sweep (Q8_0/Q4_K, M in {1,4,16,32}) with the RMSNorm
         prologue; weights rotate across distinct buffers totalling > 2x the
         256 MB Infinity Cache.
  gdn    GDN decode kernel alone (conv, L2, gates, recurrence) at B in
         {1, 8, 32, 64}, 16 heads; value = B=64 GB/s.  The decode line carries
         the same sweep as config.gdn_decode_leg.
  prefill chunked GDN prefill of one layer's core (H=16, d=128, chunks of
         64) at L=2048 and L=8192 from a zero state; value = L=8192 tokens/s,
         roofline against the f32 MFMA peak the kernels compute on.

Every timed region uses HIP events recorded on the stream the kernels are
launched on (a non-null torch stream at default priority).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
Q8_0, Q4_K = 8, 12
BPE = {Q8_0: 34 / 32, Q4_K: 144 / 256}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_threads():
    """Host cores for the CPU baseline: this process's affinity, capped by
    OMP_NUM_THREADS when set (the GPU box gives one GPU a 16-core share)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(env))) if env and env.isdigit() else n


def cpu_model():
    """The host CPU's model string (first "model name" of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# How the oracle computes a Q4_K projection row, which sets its CPU cost: the
# reference's dot_row rule (crates/zerogravity-cpu/src/source.rs:431-459).
Q4K_CPU_RULE = ("Q4_K rows by the reference's dot_row rule: serial f32 sum of (q*scale - min)*x per "
                "element, no FMA, rows spread over OpenMP threads")


def cpu_base(value, unit, cores, sample, digits=3, rule=None):
    """The cpu_baseline object: the C oracle timed on this host's cores."""
    out = {"value": round(value, digits), "unit": unit, "cores": cores, "kind": "port",
           "sample": sample, "cpu": cpu_model()}
    if rule:
        out["rule"] = rule
    return out


def gemv_bytes(kind, N, K, M):
    """Algorithmic bytes of one GEMV launch: weights once, bf16 activation
    rows in, f32 outputs out."""
    return N * K * BPE[kind] + M * K * 2 + M * N * 4


# ------------------------------------------------------------------ decode

def measured_traffic(name="decode_2b_q4k_traffic.md"):
    """HBM bytes per launch of the roofline kernel from the committed PMC
    summary (FETCH_SIZE and WRITE_SIZE passes, copy-calibrated), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def decode_matrices(g):
    """The projections one decode step streams, in launch order, as the
    resident model registers them: (label, [tensor names stacked by rows], K,
    N).  Inputs shared by several GGUF matrices are one stacked launch
    (model-qwen35/src/forward.rs layer schedule + tied LM head)."""
    H, F, V = g["hidden"], g["ffn"], g["vocab"]
    W = g["gdn_heads"] * g["gdn_dim"]
    QD, KD = g["q_heads"] * g["head_dim"], g["kv_heads"] * g["head_dim"]
    out = []
    for i in range(g["layers"]):
        p = f"blk.{i}."
        if (i + 1) % g["full_attention_interval"] == 0:
            out.append((p + "attn_in", [p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"], H,
                        2 * QD + 2 * KD))
            out.append((p + "attn_output", [p + "attn_output.weight"], QD, H))
        else:
            out.append((p + "gdn_in", [p + "attn_qkv.weight", p + "attn_gate.weight", p + "ssm_alpha.weight",
                                       p + "ssm_beta.weight"], H, 4 * W + 2 * g["gdn_heads"]))
            out.append((p + "ssm_out", [p + "ssm_out.weight"], W, H))
        out.append((p + "ffn_gate_up", [p + "ffn_gate.weight", p + "ffn_up.weight"], H, 2 * F))
        out.append((p + "ffn_down", [p + "ffn_down.weight"], F, H))
    out.append(("token_embd", ["token_embd.weight"], H, V))
    return out


def step_bytes(g, kind, B, T, tensors=None):
    """Algorithmic HBM bytes of one decode step at B rows, T cached tokens:
    every weight once (its GGUF bytes when the tensor table is given, for
    mixed codecs), GDN state read+write and conv history per row, K and V of
    T tokens (bf16) per attention layer and row, activations ignored."""
    if tensors is not None:
        w = sum(len(tensors[n][3]) for _, names, _, _ in decode_matrices(g) for n in names)
    else:
        w = sum(N * K * BPE[kind] for _, _, K, N in decode_matrices(g))
    W = g["gdn_heads"] * g["gdn_dim"]
    n_attn = g["layers"] // g["full_attention_interval"]
    n_gdn = g["layers"] - n_attn
    state = n_gdn * (g["gdn_heads"] * g["gdn_dim"] ** 2 * 4 * 2 + 3 * W * 3 * 4 * 2)
    kv = n_attn * 2 * T * g["kv_heads"] * g["head_dim"] * 2
    return w + B * (state + kv)


def run_decode(model, torch, B, prefix, steps, warmup, seed):
    """Greedy decode of `steps` positions for B rows after `warmup` untimed
    ones; tokens stay on the device (argmax output feeds the next step)."""
    from zerogravity_amd import _lib as L
    lib = L.lib()
    sess = model.session(max_batch=B, max_context=prefix + warmup + steps + 1, kv_dtype=L.BF16)
    sess.fill_random_prefix(B, prefix, seed)
    s = torch.cuda.current_stream()
    assert s.cuda_stream != 0, "launch and event stream must be a real stream"
    toks = torch.from_numpy(np.random.default_rng(seed).integers(0, model.g["vocab"], B).astype(np.int32)).cuda()
    ptr = toks.data_ptr()

    def step():
        model.ctx.check(lib.zg_decode_step_device(sess.h, B, ptr, None, ptr, s.cuda_stream))

    for _ in range(warmup):
        step()
    model.ctx.check(lib.zg_session_check(sess.h, s.cuda_stream))
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(s)
    for i in range(steps):
        step()
        ev[i + 1].record(s)
    torch.cuda.synchronize()
    model.ctx.check(lib.zg_session_check(sess.h, s.cuda_stream))
    per = np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(steps)])
    total_ms = ev[0].elapsed_time(ev[-1])
    assert sess.positions()[:B] == [prefix + warmup + steps] * B
    sess.close()
    return total_ms, per


# Prologue / epilogue codes of zg_gemv_device_fused (include/zg_hip.h)
PRO_RMS, PRO_GATED, PRO_SILU_MUL, PRO_PLAIN, PRO_GATED_PRE = 0, 1, 2, 3, 5
EPI_STORE, EPI_RESID, EPI_GLU = 0, 1, 2


def step_projections(g):
    """The B=1 decode step's projections in launch order, each with the
    prologue and epilogue the step runs it with (zg_session.hip step(), an
    all-Q4_K model): (label, [names stacked by rows], K, N, prologue,
    epilogue, role).  role: "embed" the first input projection (the token's
    embedding dequantised in its prologue), "lm" the LM head (greedy
    partials), "" otherwise."""
    H, F, V = g["hidden"], g["ffn"], g["vocab"]
    W = g["gdn_heads"] * g["gdn_dim"]
    QD, KD = g["q_heads"] * g["head_dim"], g["kv_heads"] * g["head_dim"]
    out = []
    for i in range(g["layers"]):
        p = f"blk.{i}."
        role = "embed" if i == 0 else ""
        if (i + 1) % g["full_attention_interval"] == 0:
            out.append((p + "attn_in", [p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"], H,
                        2 * QD + 2 * KD, PRO_RMS, EPI_STORE, role))
            out.append((p + "attn_output", [p + "attn_output.weight"], QD, H, PRO_PLAIN, EPI_RESID, ""))
        else:
            out.append((p + "gdn_in", [p + "attn_qkv.weight", p + "attn_gate.weight", p + "ssm_alpha.weight",
                                       p + "ssm_beta.weight"], H, 4 * W + 2 * g["gdn_heads"], PRO_RMS, EPI_STORE,
                        role))
            # (the GDN kernel forms the gated product; ssm_out applies the 1/rms)
            out.append((p + "ssm_out", [p + "ssm_out.weight"], W, H, PRO_GATED_PRE, EPI_RESID, ""))
        out.append((p + "ffn_gate_up", [p + "ffn_gate.weight", p + "ffn_up.weight"], H, 2 * F, PRO_RMS, EPI_GLU,
                    ""))
        out.append((p + "ffn_down", [p + "ffn_down.weight"], F, H, PRO_PLAIN, EPI_RESID, ""))
    out.append(("token_embd", ["token_embd.weight"], H, V, PRO_RMS, EPI_STORE, "lm"))
    return out


def gemv_leg(kern, torch, g, tensors, kind, reps):
    """The dominant kernel: the Q4_K projections of one B=1 decode step,
    replayed exactly as the step launches them -- the same stacked matrices,
    the same prologue and epilogue per projection (zg_gemv_device_fused ->
    the step's own dispatcher, so the same kernel template variants: the
    embedding prologue on the first, the gated RMSNorm's 1/rms on ssm_out
    (whose product the GDN kernel forms), SwiGLU into the down projection's
    input, residual adds, greedy partials on the
    LM head) -- captured once in a HIP graph as the step is, and the graph
    replayed `reps` times between HIP events on its stream.  ~0.95 GB per
    replay, so the weights stream from HBM, not the 256 MB Infinity Cache.
    The GDN, attention and argmax launches between them are not replayed:
    the leg times the projection kernel alone."""
    from zerogravity_amd import _lib as L
    lib, ctx = L.lib(), kern.ctx
    H, F, V = g["hidden"], g["ffn"], g["vocab"]
    W = g["gdn_heads"] * g["gdn_dim"]
    plan = step_projections(g)
    handles = {}
    embd = None
    for label, names, K, N, pro, epi, role in plan:
        parts = [tensors[n] for n in names]
        assert all(p[0] == kind and p[1] == K for p in parts), label
        h = kern.register(4243, "leg." + label, kind, K, N, np.concatenate([p[3] for p in parts]))
        handles[label] = h
        if role == "lm":
            embd = h
    rng = np.random.default_rng(7)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    ymax = max(N for _, _, _, N, _, _, _ in plan)
    bufs = dict(x=dev(rng.standard_normal(H)), x_emb=dev(np.zeros(H)), gamma=dev(1 + 0.1 * rng.standard_normal(F)),
                core=dev(rng.standard_normal(W)), z=dev(rng.standard_normal(W)),
                norm=dev(1 + 0.1 * rng.standard_normal(g["gdn_dim"])), glu=dev(rng.standard_normal(F)),
                attn=dev(rng.standard_normal(g["q_heads"] * g["head_dim"])),
                resid=dev(rng.standard_normal(H)), y=torch.empty(ymax, dtype=torch.float32, device="cuda"),
                logits=torch.empty(V, dtype=torch.float32, device="cuda"))
    tok = torch.tensor([1234], dtype=torch.int32, device="cuda")
    parts = int(lib.zg_gemv_greedy_parts(embd.h))
    gmax = torch.empty(max(parts, 1), dtype=torch.float32, device="cuda")
    gidx = torch.empty(max(parts, 1), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()

    def launch(s):
        for label, names, K, N, pro, epi, role in plan:
            h = handles[label]
            x, x2, gam, y, ldy = bufs["x"], None, bufs["gamma"], bufs["y"], N
            emb, tk, gm, gi = None, None, None, None
            if role == "embed":
                x, emb, tk = bufs["x_emb"], embd.h, tok.data_ptr()
            if label.endswith("ssm_out"):
                x, x2, gam = bufs["core"], bufs["z"], None
            elif label.endswith("attn_output"):
                x, gam = bufs["attn"], None
            elif label.endswith("ffn_down"):
                x, gam = bufs["glu"], None
            if epi == EPI_RESID:
                y, ldy = bufs["resid"], H
            elif epi == EPI_GLU:
                y, ldy = bufs["glu"], N // 2
            if role == "lm":
                y, gm, gi = bufs["logits"], gmax.data_ptr(), gidx.data_ptr()
            rc = lib.zg_gemv_device_fused(ctx.h, h.h, 1, pro, epi, x.data_ptr(), K,
                                          None if x2 is None else x2.data_ptr(), 0 if x2 is None else W,
                                          None if gam is None else gam.data_ptr(), 1e-6, g["gdn_dim"],
                                          y.data_ptr(), ldy, emb, tk, gm, gi, s.cuda_stream)
            if rc != L.COMPLETED:
                raise L.ZgError(rc, f"{label}: {ctx.error()}")

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(torch.cuda.current_stream())
    s = torch.cuda.current_stream()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        graph.replay()
    e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    byts = sum(gemv_bytes(kind, N, K, 1) for _, _, K, N, _, _, _ in plan)
    del graph
    kern.release_source(4243)
    return dict(launches=len(plan), us_per_step=us, us_per_launch=us / len(plan),
                bytes_per_launch=byts / len(plan), gbs=byts / us / 1e3)


def gdn_bytes(B, H=16, dk=128, dv=128):
    """Algorithmic bytes of one GDN decode step: the fp32 state read and
    written once, q/k/v in bf16, z in bf16 and o in f32 (per row and head)."""
    return B * H * (dk * dv * 4 * 2 + (dk + dk + dv) * 2 + dv * (2 + 4))


def gdn_leg(ctx, torch, rows=(1, 8, 32, 64), reps=20, H=16):
    """GDN decode kernel alone (conv + L2 + gates + recurrence, state
    read-modify-write) at B rows, config 3's distributions; the states rotate
    over distinct buffers totalling > 2.2x the Infinity Cache."""
    from zerogravity_amd import _lib as L
    lib = L.lib()
    s = torch.cuda.current_stream()
    out = {}
    for B in rows:
        W = H * 128
        stride = 4 * W + 2 * H
        g = torch.Generator(device="cuda")
        g.manual_seed(B)
        proj = torch.randn(B, stride, device="cuda", generator=g)
        conv_w = 0.5 * torch.randn(3 * W * 4, device="cuda", generator=g)
        dt = 0.1 * torch.randn(H, device="cuda", generator=g)
        ssm_a = -torch.exp(torch.randn(H, device="cuda", generator=g))
        ring = torch.zeros(B * 3 * W * 4, device="cuda")
        pos = torch.zeros(B, dtype=torch.int32, device="cuda")
        core = torch.empty(B * W, device="cuda")
        sbytes = B * H * 128 * 128 * 4
        copies = int(min(256, max(2, np.ceil(2.2 * MALL_BYTES / sbytes))))
        states = [0.02 * torch.randn(B * H * 128 * 128, device="cuda", generator=g) for _ in range(copies)]

        def launch(i):
            ctx.check(lib.zg_gdn_decode_device(ctx.h, B, H, proj.data_ptr(), stride, conv_w.data_ptr(),
                                               ring.data_ptr(), pos.data_ptr(), dt.data_ptr(), ssm_a.data_ptr(),
                                               1e-6, states[i % copies].data_ptr(), core.data_ptr(), s.cuda_stream))

        for i in range(copies):
            launch(i)
        torch.cuda.synchronize()
        n = max(reps, copies)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for i in range(n):
            launch(i)
        e1.record(s)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / n
        gbs = gdn_bytes(B, H) / us / 1e3
        out[B] = dict(us=round(us, 3), gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4))
        log(f"GDN decode B={B:2d}: {us:8.2f} us  {gbs:8.1f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM)")
        del states
    return out


def attn_bytes(B, T, nq=8, nkv=2, d=256):
    """Algorithmic HBM bytes of one attention decode step (one layer): K and
    V of T tokens in bf16 per row, plus q/gate in and the output out (f32)."""
    return B * (T * nkv * d * 2 * 2 + nq * d * 4 * 3)


def attn_leg(ctx, torch, rows=(1, 32), T=2048, reps=20, nq=8, nkv=2):
    """The attention decode step alone (zg_attn_decode_device: norms, RoPE,
    K/V append, scores, softmax, values, gate) at B rows, each at position
    T-1 of a bf16 cache, and its split-T form (zg_attn_decode_split_device,
    the form the decode step of an all-Q4_K model runs: span workgroups and
    the combine); the caches rotate over distinct buffers totalling > 2.2x
    the Infinity Cache."""
    from zerogravity_amd import _lib as L
    lib = L.lib()
    s = torch.cuda.current_stream()
    out = {}
    d = 256
    for B in rows:
        g = torch.Generator(device="cuda")
        g.manual_seed(100 + B)
        stride = (2 * nq + 2 * nkv) * d
        proj = torch.randn(B, stride, device="cuda", generator=g)
        qn = 1 + 0.1 * torch.randn(d, device="cuda", generator=g)
        kn = 1 + 0.1 * torch.randn(d, device="cuda", generator=g)
        pos = torch.full((B,), T - 1, dtype=torch.int32, device="cuda")
        ws = torch.empty(lib.zg_attn_decode_workspace_bytes(B, nq, T), dtype=torch.uint8, device="cuda")
        o = torch.empty(B * nq * d, device="cuda")
        cbytes = B * T * nkv * d * 2 * 2
        copies = int(min(256, max(2, np.ceil(2.2 * MALL_BYTES / cbytes))))
        caches = [(torch.randn(B * T * nkv * d, device="cuda", generator=g).bfloat16(),
                   torch.randn(B * T * nkv * d, device="cuda", generator=g).bfloat16()) for _ in range(copies)]

        sws = torch.empty(lib.zg_attn_decode_split_workspace_bytes(B, nq, nkv, T), dtype=torch.uint8, device="cuda")
        theta = float(np.power(1e7, -2.0 / 64.0))

        def launch(i, split=False):
            kc, vc = caches[i % copies]
            fn = lib.zg_attn_decode_split_device if split else lib.zg_attn_decode_device
            ctx.check(fn(ctx.h, B, nq, nkv, proj.data_ptr(), stride, qn.data_ptr(), kn.data_ptr(), 1e-6, theta,
                         pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), T, L.BF16,
                         (sws if split else ws).data_ptr(), o.data_ptr(), s.cuda_stream))

        res = {}
        for split in (False, True):
            for i in range(copies):
                launch(i, split)
            torch.cuda.synchronize()
            n = max(reps, copies)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for i in range(n):
                launch(i, split)
            e1.record(s)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / n
            gbs = attn_bytes(B, T, nq, nkv) / us / 1e3
            res[split] = (us, gbs)
            log(f"attention decode{' split-T' if split else ''} B={B:2d} T={T}: {us:8.2f} us  {gbs:8.1f} GB/s "
                f"({gbs / HBM_PEAK_GBS:.1%} of HBM)")
        (us, gbs), (sus, sgbs) = res[False], res[True]
        out[B] = dict(us=round(us, 3), gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4),
                      split_us=round(sus, 3), split_gbs=round(sgbs, 1), split_frac=round(sgbs / HBM_PEAK_GBS, 4))
        del caches
    return out


def cpu_decode_baseline(g, tensors, prefix, seconds):
    """The oracle (C restatement of the reference CPU path, OpenMP over GEMV
    rows on every host core) decoding greedily at B=1 after importing a random
    state of `prefix` tokens."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import zg_oracle as O
    threads = host_threads()
    cap = 256  # decode steps at most; the sample is bounded by `seconds` first
    model = O.Model(dict(g, max_context=prefix + cap + 2), tensors, threads)
    sess = model.session()
    n = int(sess_state_floats(g, prefix))
    rng = np.random.default_rng(3)
    sess.load_state((0.02 * rng.standard_normal(n)).astype(np.float32), prefix)
    tok = 1
    sess.forward(tok)  # first touch
    t0 = time.perf_counter()
    steps = 0
    while (time.perf_counter() - t0 < seconds or steps < 2) and steps < cap:
        tok = int(np.argmax(sess.forward(tok)))
        steps += 1
    dt = time.perf_counter() - t0
    return steps / dt, threads, f"{steps} greedy decode steps at B=1 from a random {prefix}-token state"


def sess_state_floats(g, T):
    W = g["gdn_heads"] * g["gdn_dim"]
    n_attn = g["layers"] // g["full_attention_interval"]
    n_gdn = g["layers"] - n_attn
    return n_gdn * (3 * W * 3 + g["gdn_heads"] * g["gdn_dim"] ** 2) + n_attn * 2 * T * g["kv_heads"] * g["head_dim"]


def bench_decode(args):
    import torch
    from zerogravity_amd import gguf, qwen35
    from zerogravity_amd import regions as R
    kern = R.HipMatVecKernel(0)
    torch.cuda.set_stream(torch.cuda.Stream())  # default priority, non-null
    g = dict(qwen35.QWEN35_2B)
    t0 = time.perf_counter()
    tensors = qwen35.synthetic_tensors(g, gguf.Q4_K, seed=2026)
    model = qwen35.QwenModelHip(g, tensors, kernel=kern)
    log(f"2B Q4_K model resident ({time.perf_counter() - t0:.1f} s)")
    prefix = args.prefix
    res = {}
    for B in (1, 32):
        total_ms, per = run_decode(model, torch, B, prefix, args.steps, args.warmup, seed=B)
        tps = B * args.steps / (total_ms / 1e3)
        byts = step_bytes(g, gguf.Q4_K, B, prefix + args.warmup + args.steps // 2)
        res[B] = dict(tok_s=tps, ms_per_step=total_ms / args.steps, p10_ms=float(np.percentile(per, 10)),
                      p50_ms=float(np.median(per)), p90_ms=float(np.percentile(per, 90)),
                      step_gb=byts / 1e9, step_hbm_frac=byts / (total_ms / args.steps * 1e-3) / 1e9 / HBM_PEAK_GBS)
        log(f"decode B={B:2d}: {total_ms / args.steps:.3f} ms/step  {tps:9.1f} tok/s  "
            f"(p10 {res[B]['p10_ms']:.3f} p50 {res[B]['p50_ms']:.3f} p90 {res[B]['p90_ms']:.3f} ms; "
            f"{res[B]['step_gb']:.3f} GB/step = {res[B]['step_hbm_frac']:.1%} of HBM roofline)")
    model.close()
    leg = gemv_leg(kern, torch, g, tensors, gguf.Q4_K, args.leg_reps)
    log(f"Q4_K GEMV leg: {leg['launches']} launches {leg['us_per_step']:.1f} us/step, "
        f"{leg['us_per_launch']:.2f} us/launch, {leg['gbs']:.0f} GB/s")
    gdn = gdn_leg(kern.ctx, torch)
    attn = attn_leg(kern.ctx, torch)
    line = {
        "metric": "decode tok/s @B=1 (2B-shaped Q4_K, 2048-token prefix, bf16 KV)",
        "value": round(res[1]["tok_s"], 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(res[1]["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_k weights, f32 accumulate",
        "dtype_detail": {"b1": "Q4_K codes and int16-coded activations (scale per 32-element group from its "
                               "largest magnitude, each code split into two signed bytes) on int8 MFMA, i32 "
                               "partials scaled and summed in f32",
                         "b32": "Q4_K weights dequantised to f16 tiles, f16 activations, f16 MFMA with f32 "
                                "accumulate",
                         "state": "f32 GDN state and accumulators, bf16 KV cache"},
        "data": "synthetic (seeded random-init Q4_K GGUF weights, random prefix state)",
        "config": {"workload": "2B-shaped Q4_K continuous-batch greedy decode", "prefix": prefix,
                   "kv_cache": "bf16", "b1": res[1], "b32": res[32],
                   "b32_tok_s": round(res[32]["tok_s"], 1), "gdn_decode_leg": gdn,
                   "attention_decode_leg": attn},
        "roofline": {"bound": "hbm", "achieved": round(leg["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(leg["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "gemv1_q4k_kernel (the B=1 decode step's 97 stacked Q4_K projections replayed "
                               "as the step launches them: same prologue/epilogue variants, one HIP graph)",
                     "bytes_per_launch": round(leg["bytes_per_launch"]), "us_per_launch": round(leg["us_per_launch"], 3)},
    }
    if not args.no_cpu:
        v, cores, sample = cpu_decode_baseline(g, tensors, prefix, args.cpu_seconds)
        line["cpu_baseline"] = cpu_base(v, "tok/s", cores, sample, 3, rule=Q4K_CPU_RULE)
    kern.ctx.close()
    return line


def bench_decode_q8(args, mixed=False):
    """The decode step of the 2B-shaped model with Q8_0 weights (the codec of
    the reference's pinned checkpoints): B=1, 4 and 32 greedy positions
    after a random 2048-token prefix, GEMVs in the reference's exact dot
    order (32 rows: the coded-once activation and the Q8_0 rows kernels).
    mixed: the mixed-quant layout (Q6_K embedding/LM head, V and FFN down,
    Q4_1 attention gate, F32 GDN alpha/beta) over Q8_0."""
    import torch
    from zerogravity_amd import gguf, qwen35
    from zerogravity_amd import regions as R
    kern = R.HipMatVecKernel(0)
    torch.cuda.set_stream(torch.cuda.Stream())
    g = dict(qwen35.QWEN35_2B)
    t0 = time.perf_counter()
    tensors = qwen35.synthetic_tensors(g, gguf.Q8_0, seed=2027, kinds=qwen35.MIXED if mixed else None)
    model = qwen35.QwenModelHip(g, tensors, kernel=kern)
    name = "Q8_0 + Q6_K/Q4_1/F32" if mixed else "Q8_0"
    log(f"2B {name} model resident ({time.perf_counter() - t0:.1f} s)")
    res = {}
    for B in (1, 4, 32):
        total_ms, per = run_decode(model, torch, B, args.prefix, args.steps, args.warmup, seed=B)
        ms = total_ms / args.steps
        byts = step_bytes(g, gguf.Q8_0, B, args.prefix + args.warmup + args.steps // 2, tensors if mixed else None)
        res[B] = dict(tok_s=B / ms * 1e3, ms_per_step=ms, p50_ms=float(np.median(per)), step_gb=byts / 1e9,
                      gbs=byts / ms / 1e6)
        log(f"{name} decode B={B}: {ms:.3f} ms/step  {B / ms * 1e3:8.1f} tok/s  {byts / ms / 1e6:7.0f} GB/s "
            f"({byts / ms / 1e6 / HBM_PEAK_GBS:.1%} of HBM roofline)")
    model.close()
    kern.ctx.close()
    gbs = res[1]["gbs"]
    return {
        "metric": f"decode tok/s @B=1 (2B-shaped {name}, 2048-token prefix, bf16 KV)",
        "value": round(res[1]["tok_s"], 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(res[1]["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "integer codecs, int8 dots, f32 accumulate",
        "data": f"synthetic (seeded random-init {name} GGUF weights, random prefix state)",
        "config": {"workload": f"2B-shaped {name} greedy decode", "prefix": args.prefix, "kv_cache": "bf16",
                   "b1": res[1], "b4": res[4], "b32": res[32]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole B=1 step (weights, GDN state, KV cache per step)"},
    }


# -------------------------------------------------------------------- gemv

def register_copies(kern, kind, N, K, rng):
    """Distinct device copies totalling > 2.2x the Infinity Cache."""
    from zerogravity_amd import synth
    w = synth.random_matrix(rng, kind, N, K)
    copies = int(min(512, max(2, np.ceil(2.2 * MALL_BYTES / w.nbytes))))
    return [kern.register(4242, f"bench.{kind}.{N}.{K}.{i}", kind, K, N, w) for i in range(copies)]


def bench_gemv_one(kern, torch, handles, kind, N, K, M, steps, warmup, rng, path="fused"):
    """One (codec, N, K, M) point of the sweep, rotating over the weight
    copies.  path "fused": zg_gemv_device on the f32 values of the bf16
    activation -- the decode step's kernels, the RMSNorm in their prologue
    (Q4_K: one row the int8-MFMA GEMV, from two rows the f16 activation
    tiles and the f16 MFMA GEMM, two launches; Q8_0: up to 4 rows the fused
    GEMV, beyond the coded-once activation and the rows kernels, two
    launches), all timed.
    path "prepared": the region path, the bf16 activation RMS-normalised and
    coded once (zg_act_prepare_device, untimed), then zg_gemv_prepared_device
    timed alone.  After a warm pass, `steps` launches are captured in one
    HIP graph and the graph replayed between HIP events, so the figure is
    the device's time per launch in a dependent chain, not the host's
    submission rate."""
    from zerogravity_amd import _lib as L
    from zerogravity_amd import synth
    copies = len(handles)
    xf, xb = synth.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x_d = torch.from_numpy(xb.view(np.int16)).cuda()
    x_f = torch.from_numpy(np.ascontiguousarray(xf, np.float32)).cuda()  # the same values, exactly
    g_d = torch.from_numpy(gamma).cuda()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    assert s.cuda_stream != 0, "launch and event stream must be a real stream"
    lib, ctx = L.lib(), kern.ctx
    if path == "prepared":
        nbytes = lib.zg_act_prepared_bytes(handles[0].h, M)
        prep = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        ctx.check(lib.zg_act_prepare_device(ctx.h, handles[0].h, x_d.data_ptr(), L.BF16, M, g_d.data_ptr(), 1e-6,
                                            prep.data_ptr(), nbytes, s.cuda_stream))

    def launch(i, st):
        h = handles[i % copies]
        if path == "prepared":
            ctx.check(lib.zg_gemv_prepared_device(ctx.h, h.h, M, prep.data_ptr(), y.data_ptr(), st))
        else:
            ctx.check(lib.zg_gemv_device(ctx.h, h.h, x_f.data_ptr(), L.F32, M, g_d.data_ptr(), 1e-6, y.data_ptr(),
                                         st))

    for i in range(copies):  # every copy once (a first batched call may lay out its tiles)
        launch(i, s.cuda_stream)
    for i in range(warmup):
        launch(i, s.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cs = torch.cuda.current_stream().cuda_stream
        for i in range(steps):
            launch(i, cs)
    graph.replay()
    torch.cuda.synchronize()
    reps = 4
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        graph.replay()
    e1.record(s)
    torch.cuda.synchronize()
    del graph
    us = e0.elapsed_time(e1) * 1e3 / (steps * reps)
    return us, gemv_bytes(kind, N, K, M) / us / 1e3


def cpu_gemv_baseline(kind, N, K, seconds):
    """Oracle GEMV (OpenMP over rows, all host cores) on a bounded row sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import zg_oracle as O
    from zerogravity_amd import synth
    rng = np.random.default_rng(1)
    rows = min(N, 32768)
    w = synth.random_matrix(rng, kind, rows, K)
    x = rng.standard_normal(K).astype(np.float32)
    threads = host_threads()
    O.matvec(kind, w.reshape(-1), rows, K, x, threads)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        O.matvec(kind, w.reshape(-1), rows, K, x, threads)
        n += 1
    dt = (time.perf_counter() - t0) / n
    byts = rows * K * BPE[kind] + K * 4 + rows * 4
    return byts / dt / 1e9, threads, f"{rows}x{K} rows of the {N}x{K} matrix, {n} passes"


def bench_gemv(args):
    import torch
    from zerogravity_amd import regions as R
    kern = R.HipMatVecKernel(0)
    torch.cuda.set_stream(torch.cuda.Stream())
    rng = np.random.default_rng(2026)
    results = []
    shapes = [(3584, 1024), (1024, 3584), (6144, 2048), (2048, 6144), (151936, 2048)]
    for kind in (Q4_K, Q8_0):
        for (N, K) in shapes:
            handles = register_copies(kern, kind, N, K, rng)
            for M in (1, 4, 16, 32):
                for path in ("fused", "prepared"):
                    us, gbs = bench_gemv_one(kern, torch, handles, kind, N, K, M, args.steps, args.warmup, rng,
                                             path)
                    name = "Q4_K" if kind == Q4_K else "Q8_0"
                    log(f"gemv {name} N={N:6d} K={K:5d} M={M:2d} {path:>8}: {us:9.2f} us  {gbs:8.1f} GB/s  "
                        f"({gbs / HBM_PEAK_GBS:.1%} of HBM)")
                    results.append(dict(kind=name, N=N, K=K, M=M, path=path, us=round(us, 3), gbs=round(gbs, 1)))
            del handles
            kern.release_source(4242)
    head = next(r for r in results if r["kind"] == "Q4_K" and r["N"] == 151936 and r["M"] == 1
                and r["path"] == "fused")
    line = {
        "metric": "dequant-GEMV achieved HBM GB/s (Q4_K 151936x2048, M=1, fused RMSNorm prologue)",
        "value": head["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["us"] / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k x f32", "data": "synthetic (seeded random GGUF blocks)",
        "config": {"workload": "dequant-GEMV sweep", "sweep": results},
        "roofline": {"bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
    }
    if not args.no_cpu:
        v, cores, sample = cpu_gemv_baseline(Q4_K, 151936, 2048, args.cpu_seconds)
        line["cpu_baseline"] = cpu_base(v, "GB/s", cores, sample, 2, rule=Q4K_CPU_RULE)
    kern.ctx.close()
    return line


# ----------------------------------------------------------------- prefill

F32_MFMA_PEAK_TFLOPS = 157.3
F16_MFMA_PEAK_TFLOPS = 2500.0  # dense f16 MFMA (no sparsity)
PREFILL_C, PREFILL_D = 64, 128


def prefill_flops_per_chunk_head():
    """Algorithmic multiply-adds of one 64-token chunk of one head (C = 64,
    d = 128), counted as the chunk reference computes them
    (numerics/torch_cpu/gdn/chunk/core.rs:152-274): A and intra (C x C x d
    each, full squares), the two unit-lower solves (C(C-1)/2 x d each), W S
    and dq S (C x d x d each), intra corr (C x d x C) and the state update
    dk^T corr (d x d x C).  Two flops per multiply-add."""
    C, d = PREFILL_C, PREFILL_D
    macs = 2 * C * C * d + 2 * (C * (C - 1) // 2) * d + 2 * C * d * d + C * d * C + d * d * C
    return 2 * macs


def prefill_inputs(torch, T, H, seed):
    """Config 4's synthetic distribution on the device: bf16-exact q, k, v,
    beta = sigmoid(N(0,1)) (bf16-exact), log decay = -softplus(N(0,1)) *
    exp(N(0,0.5)), zero initial state."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    n = T * H * PREFILL_D
    q, k, v = (torch.randn(n, device="cuda", generator=g).bfloat16().float() for _ in range(3))
    beta = torch.sigmoid(torch.randn(T * H, device="cuda", generator=g)).bfloat16().float()
    a, b = torch.randn(T * H, device="cuda", generator=g), torch.randn(T * H, device="cuda", generator=g)
    logd = (-torch.nn.functional.softplus(a) * torch.exp(0.5 * b)).clamp(max=0.0)
    return q, k, v, beta, logd


def cpu_prefill_baseline(T, H, seconds):
    """The oracle's chunk prefill (one host thread) on L = T tokens of H heads."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import zg_oracle as O
    rng = np.random.default_rng(3)
    n = T * H * PREFILL_D
    q, k, v = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    beta = (1 / (1 + np.exp(-rng.standard_normal(T * H)))).astype(np.float32)
    logd = (-np.log1p(np.exp(rng.standard_normal(T * H)))).astype(np.float32)
    t0 = time.perf_counter()
    reps = 0
    while True:
        O.gdn_chunk_prefill(q, k, v, beta, logd, H, PREFILL_D, PREFILL_C)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    return T / dt, 1, f"L={T} tokens x {H} heads, {reps} pass(es) of the oracle chunk prefill"


def bench_prefill(args):
    import torch
    from zerogravity_amd import _lib as L
    from zerogravity_amd import chunk as CH
    ctx = L.Context(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    H = 16
    results = []
    for T in (2048, 8192):
        q, k, v, beta, logd = prefill_inputs(torch, T, H, 4 + T)
        state = torch.zeros(H * PREFILL_D * PREFILL_D, device="cuda")
        out = torch.empty(T * H * PREFILL_D, device="cuda")
        torch.cuda.synchronize()

        def launch():
            state.zero_()
            CH.prefill_device(ctx, T, H, q, k, v, beta, logd, state, out, stream.cuda_stream)

        for _ in range(args.warmup):
            launch()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        chunks = (T + PREFILL_C - 1) // PREFILL_C
        tflops = chunks * H * prefill_flops_per_chunk_head() / (ms * 1e-3) / 1e12
        log(f"prefill L={T} H={H}: {ms * 1e3:9.1f} us/call  {T / ms * 1e3:12.0f} tok/s  {tflops:7.2f} TFLOP/s "
            f"({tflops / F32_MFMA_PEAK_TFLOPS:.1%} of f32 MFMA peak)")
        results.append(dict(L=T, H=H, us=round(ms * 1e3, 2), tok_s=round(T / ms * 1e3, 1),
                            tflops=round(tflops, 3)))
    head = results[-1]
    line = {
        "metric": "chunked GDN prefill tokens/s (one GDN layer's core, L=8192, H=16, d=128, C=64)",
        "value": head["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["us"] / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded bf16-exact q/k/v, sigmoid beta, softplus decay)",
        "config": {"workload": "chunked GDN prefill", "sweep": results},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": F32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(head["tflops"] / F32_MFMA_PEAK_TFLOPS, 4), "traffic": None},
    }
    if not args.no_cpu:
        v, cores, sample = cpu_prefill_baseline(2048, H, args.cpu_seconds)
        line["cpu_baseline"] = cpu_base(v, "tok/s", cores, sample, 2)
    ctx.close()
    return line


def model_prefill_flops(g, L):
    """Algorithmic flops of one batched prefill of L tokens: every projection
    once per token (2 N K), the GDN chunk cores (prefill_flops_per_chunk_head
    per 64-token chunk and head), causal attention (QK and PV over t + 1 keys
    for token t, every query head) and the LM head of the last token."""
    proj = sum(N * K for _, _, K, N in decode_matrices(g)[:-1])
    n_attn = g["layers"] // g["full_attention_interval"]
    n_gdn = g["layers"] - n_attn
    chunks = (L + PREFILL_C - 1) // PREFILL_C
    gdn = n_gdn * chunks * g["gdn_heads"] * prefill_flops_per_chunk_head()
    attn = n_attn * g["q_heads"] * 2 * 2 * g["head_dim"] * (L * (L + 1) // 2)
    return 2 * proj * L + gdn + attn + 2 * g["vocab"] * g["hidden"]


def cpu_model_prefill_baseline(g, tensors, seconds):
    """The oracle's per-token prefill (QwenDenseCpu::prefill_transaction,
    OpenMP over GEMV rows on every host core) on a bounded prompt."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import zg_oracle as O
    threads = host_threads()
    model = O.Model(dict(g, max_context=1024), tensors, threads)
    sess = model.session()
    toks = np.random.default_rng(5).integers(0, g["vocab"], 1000)
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0 < seconds or n < 2) and n < len(toks):
        sess.forward(int(toks[n]), need_logits=n == len(toks) - 1)
        n += 1
    dt = time.perf_counter() - t0
    return n / dt, threads, f"{n} prompt tokens through the per-token prefill"


def bench_model_prefill(args):
    """Batched prefill of one prompt on the 2B-shaped Q4_K model
    (zg_prefill_batched), L = 512, 2048 and 8192; each timed call starts from
    a reset session (the reset is outside the timed region)."""
    from zerogravity_amd import _lib as L
    from zerogravity_amd import gguf, qwen35
    from zerogravity_amd import regions as R
    kern = R.HipMatVecKernel(0)
    g = dict(qwen35.QWEN35_2B)
    tensors = qwen35.synthetic_tensors(g, gguf.Q4_K, seed=2026)
    model = qwen35.QwenModelHip(g, tensors, kernel=kern)
    rng = np.random.default_rng(7)
    steps = max(1, min(args.steps, 16))
    results = []
    for T in (512, 2048, 8192):
        sess = model.session(max_batch=1, max_context=T, kv_dtype=L.BF16)
        toks = rng.integers(0, g["vocab"], T).astype(np.uint32)
        for _ in range(max(1, min(args.warmup, 2))):
            sess.reset()
            sess.prefill_batched(toks)
        total = 0.0
        for _ in range(steps):
            sess.reset()
            t0 = time.perf_counter()
            sess.prefill_batched(toks)  # returns after the logits reach the host
            total += time.perf_counter() - t0
        sess.close()
        ms = total / steps * 1e3
        tflops = model_prefill_flops(g, T) / (ms * 1e-3) / 1e12
        log(f"model prefill L={T}: {ms:8.2f} ms  {T / ms * 1e3:10.0f} tok/s  {tflops:7.1f} TFLOP/s "
            f"({tflops / F16_MFMA_PEAK_TFLOPS:.1%} of f16 MFMA peak)")
        results.append(dict(L=T, ms=round(ms, 3), tok_s=round(T / ms * 1e3, 1), tflops=round(tflops, 2)))
    model.close()
    head = results[1]
    line = {
        "metric": "batched prefill tok/s (2B-shaped Q4_K, 2048-token prompt, bf16 KV)",
        "value": head["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": head["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k weights, f16 MFMA, f32 accumulate",
        "data": "synthetic (seeded random-init Q4_K GGUF weights, random prompt ids)",
        "config": {"workload": "2B-shaped Q4_K batched prefill of one row", "sweep": results},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(head["tflops"] / F16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "whole prefill (all kernels; algorithmic flops / wall time)"},
    }
    if not args.no_cpu:
        v, cores, sample = cpu_model_prefill_baseline(g, tensors, args.cpu_seconds)
        line["cpu_baseline"] = cpu_base(v, "tok/s", cores, sample, 2, rule=Q4K_CPU_RULE)
    kern.ctx.close()
    return line


def bench_copy(args):
    """A plain device copy of 256 MiB (one elementwise kernel reading and
    writing 256 MiB): the calibration for the FETCH_SIZE / WRITE_SIZE
    counters and a check of the achievable read+write bandwidth."""
    import torch
    n = (256 << 20) // 4
    a = torch.randn(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(max(1, args.warmup)):
        torch.add(a, 0.0, out=b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    steps = max(1, args.steps)
    e0.record()
    for _ in range(steps):
        torch.add(a, 0.0, out=b)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    gbs = 2 * n * 4 / us / 1e3
    log(f"copy 256 MiB: {us:.1f} us  {gbs:.0f} GB/s read+write")
    del a, b
    ceilings = bandwidth_ceilings(torch) if args.ceilings else None
    return {"metric": "device copy GB/s (256 MiB read + 256 MiB written)", "value": round(gbs, 1), "unit": "GB/s",
            "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(us / 1e3, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "calibration copy", "bytes_read": n * 4, "bytes_written": n * 4,
                       "ceilings_gbs": ceilings}}


def bandwidth_ceilings(torch, reps=20):
    """Read + write bandwidth of this box for the two patterns the GDN decode
    state can take: a copy (read one buffer, write another: the double-
    buffered state of a session step) and an in-place read-modify-write (the
    region entry's state).  One vectorised elementwise kernel per buffer,
    rotating over buffers totalling more than 1 GiB so that nothing is served
    from the 256 MB Infinity Cache; GB/s counts bytes read plus written."""
    out = {"copy": {}, "rmw": {}}
    for mib in (16, 64, 256):
        n = (mib << 20) // 4
        k = max(2, (1024 // mib) + 1)
        src = [torch.randn(n, device="cuda") for _ in range(k)]
        dst = [torch.empty_like(src[0]) for _ in range(k)]
        for kind in ("copy", "rmw"):
            def run(i):
                if kind == "copy":
                    torch.mul(src[i % k], 1.0001, out=dst[i % k])
                else:
                    src[i % k].mul_(0.9999)
            for i in range(k):
                run(i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(reps * k):
                run(i)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * k)
            out[kind][f"{mib}MiB"] = round(2 * n * 4 / us / 1e3, 1)
            log(f"{kind} {mib} MiB: {us:.1f} us  {out[kind][f'{mib}MiB']:.0f} GB/s read+write")
        del src, dst
    return out


def cpu_gdn_baseline(seconds, H=16):
    """The oracle's GDN decode step at B=1 (conv over 3 x 2048 channels, SiLU,
    two-stage q/k L2, gates, the 16-head recurrence; one host thread, serial
    per head as host_math.rs:1007-1016 runs it)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import zg_oracle as O
    rng = np.random.default_rng(9)
    W, D = H * 128, 128
    conv_w = (0.5 * rng.standard_normal(3 * W * 4)).astype(np.float32)
    hist = np.zeros(3 * W * 3, np.float32)
    state = (0.02 * rng.standard_normal(H * D * D)).astype(np.float32)
    dt, a = rng.standard_normal(H).astype(np.float32), -np.exp(rng.standard_normal(H)).astype(np.float32)
    sc = np.full(D, 1.0 / np.sqrt(np.float32(D)), np.float32)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds or n < 2:
        x = rng.standard_normal(4 * W + 2 * H).astype(np.float32)
        raw, hist = O.gdn_conv_step(x[:3 * W], conv_w, hist)
        mixed = O.silu(raw)
        gain, beta = O.gdn_coefficients(x[4 * W:4 * W + H], x[4 * W + H:], dt, a, 1.0 / np.sqrt(D))[:2]
        qk = O.grouped_rms_norm(mixed[:2 * W], sc, 2 * H, 1e-6 / D)
        for h in range(H):
            o, state[h * D * D:(h + 1) * D * D] = O.gdn_recurrent_step(
                state[h * D * D:(h + 1) * D * D], qk[h * D:(h + 1) * D], qk[W + h * D:W + (h + 1) * D],
                mixed[2 * W + h * D:2 * W + (h + 1) * D], float(gain[h]), float(beta[h]), 1.0 / np.sqrt(D))
        n += 1
    dt_s = (time.perf_counter() - t0) / n
    return gdn_bytes(1, H) / dt_s / 1e9, 1, f"{n} GDN decode steps at B=1 (16 heads) through the oracle"


def bench_gdn(args):
    import torch
    from zerogravity_amd import _lib as L
    ctx = L.Context(0)
    torch.cuda.set_stream(torch.cuda.Stream())
    res = gdn_leg(ctx, torch, reps=max(args.steps, 20))
    head = res[64]
    line = {
        "metric": "GDN decode achieved HBM GB/s (B=64, 16 heads, dk=dv=128, fp32 state read-modify-write)",
        "value": head["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": max(args.steps, 20), "warmup": 1,
        "ms_per_step": head["us"] / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded projections, N(0,0.02) states)",
        "config": {"workload": "GDN decode step (conv + L2 + gates + recurrence)", "sweep": res},
        "roofline": {"bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["frac"], "traffic": None},
    }
    if not args.no_cpu:
        v, cores, sample = cpu_gdn_baseline(min(args.cpu_seconds, 10.0))
        line["cpu_baseline"] = cpu_base(v, "GB/s", cores, sample, 3)
    ctx.close()
    return line


def bench_config1(args):
    """Config 1: the 0.8B-shaped Q8_0 model, 32 seeded prompt ids through the
    per-token prefill and 32 greedy decode steps at B=1 (tokens and logits
    through the host API, as QwenDenseCpu runs it); the oracle runs the same
    request on the host cores."""
    from zerogravity_amd import _lib as L
    from zerogravity_amd import gguf, qwen35
    from zerogravity_amd import regions as R
    kern = R.HipMatVecKernel(0)
    g = dict(qwen35.QWEN35_0_8B)
    tensors = qwen35.synthetic_tensors(g, gguf.Q8_0, seed=2025)
    model = qwen35.QwenModelHip(g, tensors, kernel=kern)
    prompt = np.random.default_rng(1).integers(0, g["vocab"], 32).astype(np.uint32)
    times = []
    for _ in range(max(1, min(args.steps, 5))):
        sess = model.session(max_batch=1, max_context=128, kv_dtype=L.F32)
        t0 = time.perf_counter()
        lg = sess.prefill_transaction(prompt)
        toks = []
        for _ in range(32):
            t = int(np.argmax(lg))
            toks.append(t)
            lg = sess.forward(t)
        times.append(time.perf_counter() - t0)
        sess.close()
    model.close()
    sec = float(np.median(times))
    line = {
        "metric": "config-1 request tok/s (0.8B-shaped Q8_0, 32 prompt + 32 greedy tokens, B=1)",
        "value": round(64 / sec, 1), "unit": "tok/s", "n_gpus": 1, "steps": len(times), "warmup": 0,
        "ms_per_step": round(sec * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q8_0 weights, int8 dot, f32 accumulate",
        "data": "synthetic (seeded random-init Q8_0 GGUF weights, seeded prompt ids)",
        "config": {"workload": "config 1 end to end (host API per token)", "greedy": toks[:8]},
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import zg_oracle as O
        threads = host_threads()
        o = O.Model(dict(g, max_context=128), tensors, threads).session()
        t0 = time.perf_counter()
        n = 0
        for t in prompt:
            o.forward(int(t), need_logits=n == 31)
            n += 1
            if time.perf_counter() - t0 > args.cpu_seconds:
                break
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = cpu_base(n / dt, "tok/s", threads, f"{n} prompt tokens of the same request through the oracle", 3)
    kern.ctx.close()
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "decode_q8", "decode_mixed", "gemv", "prefill", "gdn", "model_prefill", "copy", "config1"])
    ap.add_argument("--prefix", type=int, default=2048)
    ap.add_argument("--leg-reps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ceilings", action="store_true",
                    help="copy workload: also the copy and in-place read-modify-write ceilings at 16-256 MiB")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (batch rows are independent and "
              "the weights replicate, so each GPU would run its own sessions)", file=sys.stderr)
        sys.exit(2)
    bench = {"decode": bench_decode, "decode_q8": bench_decode_q8,
             "decode_mixed": lambda a: bench_decode_q8(a, mixed=True), "gemv": bench_gemv, "prefill": bench_prefill, "gdn": bench_gdn,
             "model_prefill": bench_model_prefill, "copy": bench_copy, "config1": bench_config1}[args.workload]
    line = bench(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
