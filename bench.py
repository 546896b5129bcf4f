"""Throughput of libkk's op classes on one MI355X.

A step is one pass of the reduction workload over one set of resident
inputs: AdaIN (InstanceNorm over T, eps 1e-5, with the style Linear
128 -> 1024 fused) on [1,512,1200] and on [1,512,9600], LayerNorm(768,
eps 1e-12) on [1,256,768] and Softmax(last axis) on [1,12,256,256].  `value`
is the algorithmic HBM bytes of a step divided by its time (GB/s).

The second half of the metric, audio-seconds per wall-second, is the
`kokoro_graph` object: the whole packed Kokoro graph for 128 phoneme ids,
timed from host ids to host waveform.

Timing: every step's kernels are recorded once into a HIP graph per input
set; the timed region replays them with HIP events on libkk's stream.
Inputs rotate over enough sets (> 512 MB) that the 256 MB Infinity Cache
cannot serve them.  Per-op lines (elementwise set, reductions, dequant
GEMM/conv, the decoder upsample stage) are measured the same way, one op
per graph node.  The CPU baseline runs the numpy oracle on this host.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-graph]
                       [--no-output-stage] [--graph-ids 128] [--graph-reps 5]
                       [--graph-cpu-ids 2]
"""
import argparse
import ctypes
import importlib
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("achieved HBM GB/s (% of peak) per op class; audio-sec per wall-sec on "
          "Kokoro graph")
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
FP32_PEAK_TFLOPS = 157.3    # MI355X dense fp32 (vector and MFMA)
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA
ROTATE_BYTES = 640 << 20    # > 2x the 256 MB Infinity Cache
# Matrix-core paths of the contraction lines: (description, effective peak
# in TFLOP/s of fp32-accurate work) from MI355X's dense peaks (bf16/fp16
# 2.5 PFLOP/s, int8 5.0 POPS, fp32 157.3 TFLOP/s) and the MFMAs per product.
MFMA_PEAKS = {
    "fp32": ("fp32 MFMA (v_mfma_f32_16x16x4_f32)", 157.3),
    "bf16x3": ("bf16 MFMA, activations in 3 bf16 parts (v_mfma_f32_32x32x16_bf16 x3)", 2500.0 / 3),
    "bf16x6": ("bf16 MFMA, activations in 3 bf16 parts, fp16 weights in 2 "
               "(v_mfma_f32_32x32x16_bf16 x6)", 2500.0 / 6),
    "f16x2": ("fp16 MFMA, activations in 2 fp16 parts (v_mfma_f32_32x32x16_f16 x2)", 1250.0),
    "i8": ("int8 MFMA (v_mfma_i32_32x32x32_i8)", INT8_PEAK_TOPS),
}


GRAPH_REPEAT = 4  # calls of an op per rotating input set in a per-op timing graph (--graph-repeat)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Bench:
    def __init__(self, kk):
        self.kk = kk
        self.lib = kk._lib
        self.D = kk.to_device

    def call(self, name, *args):
        self.lib.call(name, *args)

    def graph(self, fn):
        """Record fn()'s launches into a HIP graph; returns its id."""
        self.call("kk_graph_begin")
        try:
            fn()
        except Exception:
            gid = ctypes.c_int()
            self.lib.load().kk_graph_end(ctypes.byref(gid))
            raise
        gid = ctypes.c_int()
        self.call("kk_graph_end", ctypes.byref(gid))
        return gid.value

    def time_graphs(self, gids, reps):
        """Average ms per replay of the list `gids` launched in turn."""
        for g in gids:  # warm
            self.call("kk_graph_launch", g)
        self.kk.sync()
        self.call("kk_event_record", 0)
        for _ in range(reps):
            for g in gids:
                self.call("kk_graph_launch", g)
        self.call("kk_event_record", 1)
        ms = ctypes.c_float()
        self.call("kk_event_elapsed", 0, 1, ctypes.byref(ms))
        return ms.value / (reps * len(gids))

    def graph_nodes(self, gid):
        n = ctypes.c_int64()
        self.call("kk_graph_nodes", gid, ctypes.byref(n))
        return int(n.value)

    def kernels_per_call(self, fn, i=0):
        """Kernels one eager call of fn(i) launches (libkk's dispatch count)."""
        before = self.kk.dispatch_count()
        fn(i)
        return self.kk.dispatch_count() - before

    def time_eager(self, fn, sets, reps):
        """Average ms per call of fn(i) for i in range(sets), called eagerly
        (for ops that draw scratch from the pool, which a graph recording
        does not allow)."""
        for i in range(sets):  # warm (pool blocks, code objects)
            fn(i)
        self.kk.sync()
        self.call("kk_event_record", 0)
        for _ in range(reps):
            for i in range(sets):
                fn(i)
        self.call("kk_event_record", 1)
        ms = ctypes.c_float()
        self.call("kk_event_elapsed", 0, 1, ctypes.byref(ms))
        return ms.value / (reps * sets)

    def replicate(self, t, n):
        """n device copies of t (device-to-device)."""
        out = [t]
        for _ in range(n - 1):
            c = self.kk.DeviceTensor.empty(t.shape, t.dtype)
            self.kk.ops.copy_into(c, t)
            out.append(c)
        return out


# ------------------------------------------------------------ workloads
def reduction_inputs(seed=0):
    """Seeded like the parity tests: x ~ N(0,1), style ~ N(0,0.1) [1,128],
    W ~ N(0,0.05) [128,1024], b = 0; LN gamma = 1 + 0.1N, beta = 0.1N;
    softmax input ~ N(0, std 2)."""
    r = np.random.default_rng(seed)
    return dict(
        x1200=r.normal(0, 1, (1, 512, 1200)).astype(np.float32),
        x9600=r.normal(0, 1, (1, 512, 9600)).astype(np.float32),
        style=r.normal(0, 0.1, (1, 128)).astype(np.float32),
        w=r.normal(0, 0.05, (128, 1024)).astype(np.float32),
        b=np.zeros(1024, np.float32),
        ln=r.normal(0, 1, (1, 256, 768)).astype(np.float32),
        g=(1 + 0.1 * r.normal(0, 1, 768)).astype(np.float32),
        beta=(0.1 * r.normal(0, 1, 768)).astype(np.float32),
        sm=r.normal(0, 2, (1, 12, 256, 256)).astype(np.float32),
    )


def adain_bytes(c, t, s=128):
    # read x, write y, read W [S,2C], style [S], bias [2C]
    return 2 * c * t * 4 + s * 2 * c * 4 + s * 4 + 2 * c * 4


BYTES = {
    "adain_t1200": adain_bytes(512, 1200),
    "adain_t9600": adain_bytes(512, 9600),
    "layernorm_768": 2 * 256 * 768 * 4 + 2 * 768 * 4,
    "softmax_12x256x256": 2 * 12 * 256 * 256 * 4,
}
STEP_BYTES = sum(BYTES.values())


def pmc_traffic(kernel):
    """HBM bytes per launch of `kernel` measured by the FETCH_SIZE and
    WRITE_SIZE counter runs summarised in profiles/ (null until measured)."""
    path = os.path.join(ROOT, "profiles", "instnorm_adain_t9600_hbm_traffic.md")
    try:
        text = open(path).read()
    except OSError:
        return None
    for line in text.splitlines():
        if line.startswith(f"traffic_bytes_per_launch {kernel} = "):
            return int(line.rsplit("=", 1)[1])
    return None


def output_stage_lines(kk, B, D, r, per_op):
    """Bench lines of the output stage: the 1023-tap notch FIR, PCM16, and
    both fused, over a 2,154,000-sample waveform (rotating sets)."""
    aud = importlib.import_module("best-tts-godot_amd.audio")
    ns = 2154000
    na = max(2, -(-ROTATE_BYTES // (6 * ns)))
    wav = B.replicate(D((0.25 * r.normal(0, 1, ns)).astype(np.float32)), na)
    taps = D(aud.notch_taps())
    ntap = int(taps.shape[0])
    wout = [kk.DeviceTensor.empty((ns,)) for _ in range(na)]
    pout = [kk.DeviceTensor.empty((2 * ns,), np.uint8) for _ in range(na)]
    per_op("fir_notch_1023_x2154000", lambda i: B.call(
        "kk_fir", wout[i].desc(), wav[i].desc(), taps.desc(), -1), flops=2 * ntap * ns, sets=na,
        reps=5)
    per_op("pcm16_x2154000", lambda i: B.call("kk_pcm16", pout[i].desc(), wav[i].desc(), 1.0),
                 6 * ns, sets=na)
    per_op("fir_pcm16_x2154000", lambda i: B.call(
        "kk_fir_pcm16", pout[i].desc(), wav[i].desc(), taps.desc(), -1, 1.0), 6 * ns,
        flops=2 * ntap * ns, sets=na, reps=5)
    del wav, wout, pout


def run_gpu(args):
    kk = importlib.import_module("best-tts-godot_amd")
    kk.init(0)
    B = Bench(kk)
    D = B.D
    host = reduction_inputs()
    nsets = max(2, -(-ROTATE_BYTES // (2 * STEP_BYTES)))  # inputs + outputs per set
    log(f"bench: {nsets} rotating sets x {2 * STEP_BYTES / 1e6:.1f} MB")
    # The style Linear's W [128, 1024] is kept as W^T in memory (a transposed
    # view): each channel's gamma and beta columns are then contiguous.
    style, b = D(host["style"]), D(host["b"])
    w = D(np.ascontiguousarray(host["w"].T)).transpose([1, 0])
    g, beta = D(host["g"]), D(host["beta"])
    xs = {k: B.replicate(D(host[k]), nsets) for k in ("x1200", "x9600", "ln", "sm")}
    outs = {k: [kk.DeviceTensor.empty(v[0].shape) for _ in range(nsets)] for k, v in xs.items()}
    eps_in, eps_ln = 1e-5, 1e-12

    def op_adain(k, i):
        B.call("kk_adain", outs[k][i].desc(), xs[k][i].desc(), style.desc(), w.desc(), None, None,
               b.desc(), eps_in)

    def op_ln(i):
        B.call("kk_layernorm", outs["ln"][i].desc(), xs["ln"][i].desc(), None, None, g.desc(),
               beta.desc(), -1, eps_ln)

    def op_sm(i):
        B.call("kk_softmax", outs["sm"][i].desc(), xs["sm"][i].desc(), -1)

    def step(i):
        op_adain("x1200", i)
        op_adain("x9600", i)
        op_ln(i)
        op_sm(i)

    # The W warm-up steps and the K timed steps are each one recorded graph
    # of exactly that many steps, walking the rotating input sets in turn, so
    # the timed region is one graph launch whatever K is.
    def steps_graph(k_steps, first=0):
        return B.graph(lambda: [step((first + j) % nsets) for j in range(k_steps)])

    timed = steps_graph(args.steps, args.warmup)
    if args.warmup > 0:
        warm = steps_graph(args.warmup)
        B.call("kk_graph_launch", warm)
        kk.sync()
        B.call("kk_graph_destroy", warm)
    kk.sync()
    B.call("kk_event_record", 2)
    B.call("kk_graph_launch", timed)
    B.call("kk_event_record", 3)
    kk.sync()
    ms = ctypes.c_float()
    B.call("kk_event_elapsed", 2, 3, ctypes.byref(ms))
    B.call("kk_graph_destroy", timed)
    ms_per_step = ms.value / args.steps
    log(f"bench: step {ms_per_step * 1e3:.2f} us ({STEP_BYTES / ms_per_step / 1e6:.0f} GB/s)")

    # ---- per-op lines: one graph per set, each with a single op node
    ops_out = {}

    def per_op(name, fn, nbytes=None, flops=None, reps=20, sets=nsets, eager=False, mfma=None):
        if eager:
            t_ms = B.time_eager(fn, sets, reps)
            kernels = B.kernels_per_call(fn)
        else:  # one graph holding the op GRAPH_REPEAT times per rotating set
            # (each replay's own launch cost spread over as many calls as a
            # graph of a few ops would; the model graph holds thousands)
            gid = B.graph(lambda: [fn(i) for _ in range(GRAPH_REPEAT) for i in range(sets)])
            t_ms = B.time_graphs([gid], reps) / (sets * GRAPH_REPEAT)
            kernels = B.graph_nodes(gid) / (sets * GRAPH_REPEAT)
            B.call("kk_graph_destroy", gid)
        rec = {"us": round(t_ms * 1e3, 3), "kernels": kernels}
        if nbytes:
            gbs = nbytes / (t_ms * 1e-3) / 1e9
            rec.update(bytes=nbytes, gbps=round(gbs, 1), frac_hbm=round(gbs / HBM_PEAK_GBS, 4))
        if flops:
            tf = flops / (t_ms * 1e-3) / 1e12
            rec.update(flops=flops, tflops=round(tf, 2))
            if mfma != "i8":  # fp32-semantics work: its fraction of the fp32 peak
                rec["frac_fp32"] = round(tf / FP32_PEAK_TFLOPS, 4)
            if mfma:  # the matrix-core type the kernel runs on, at its effective peak
                kind, peak = MFMA_PEAKS[mfma]
                rec.update(mfma=kind, mfma_peak_tflops=peak, frac_mfma=round(tf / peak, 4))
        ops_out[name] = rec
        log(f"bench: {name:<28} {json.dumps(rec)}")
        return rec

    # A plain fp32 copy of each reduction's input (read + write of the same
    # bytes): the bandwidth a kernel of that size can reach at all (launch
    # and ramp dominate at a few MB), each op's frac_of_copy against it; the
    # T=9600 copy is also the calibration kernel for the HBM byte counters.
    copies = {}
    for key, tag in (("x1200", "512x1200"), ("x9600", "512x9600"), ("ln", "256x768"),
                     ("sm", "12x256x256")):
        copies[key] = per_op(f"copy_{tag}", lambda i, k=key: B.call(
            "kk_copy", outs[k][i].desc(), xs[k][i].desc()), 2 * 4 * xs[key][0].size)
    cp = copies["x9600"]

    def vs_copy(rec, key):
        rec["frac_of_copy"] = round(rec["gbps"] / copies[key]["gbps"], 4)
        return rec

    vs_copy(per_op("adain_t1200", lambda i: op_adain("x1200", i), BYTES["adain_t1200"]), "x1200")
    dom = vs_copy(per_op("adain_t9600", lambda i: op_adain("x9600", i), BYTES["adain_t9600"]), "x9600")
    vs_copy(per_op("layernorm_768", op_ln, BYTES["layernorm_768"]), "ln")
    vs_copy(per_op("softmax_12x256x256", op_sm, BYTES["softmax_12x256x256"]), "sm")

    # elementwise set: x [1,512,2400], per-channel c, alpha
    r = np.random.default_rng(0)
    ex = D(r.normal(0, 1, (1, 512, 2400)).astype(np.float32))
    ec = D(r.normal(0, 1, (1, 512, 1)).astype(np.float32))
    ea = D(r.uniform(0.5, 2, (1, 512, 1)).astype(np.float32))
    ne = max(2, -(-ROTATE_BYTES // (2 * 4915200)))
    exs = B.replicate(ex, ne)
    eos = [kk.DeviceTensor.empty(ex.shape) for _ in range(ne)]
    ebytes = 2 * 4915200 + 2048
    opc = kk._lib.OP
    copies["e"] = per_op("copy_1x512x2400", lambda i: B.call("kk_copy", eos[i].desc(), exs[i].desc()),
                         2 * 4915200, sets=ne)
    vs_copy(per_op("add_1x512x2400", lambda i: B.call("kk_binary", opc["Add"], eos[i].desc(),
                                                       exs[i].desc(), ec.desc()), ebytes, sets=ne), "e")
    vs_copy(per_op("mul_1x512x2400", lambda i: B.call("kk_binary", opc["Mul"], eos[i].desc(),
                                                       exs[i].desc(), ec.desc()), ebytes, sets=ne), "e")
    vs_copy(per_op("leakyrelu_1x512x2400", lambda i: B.call("kk_unary", opc["LeakyRelu"], eos[i].desc(),
                                                             exs[i].desc(), 0.2), 2 * 4915200, sets=ne), "e")
    vs_copy(per_op("snake_1x512x2400", lambda i: B.call("kk_snake", eos[i].desc(), exs[i].desc(),
                                                         ea.desc(), None), ebytes, sets=ne), "e")
    del exs, eos

    # The same op classes at the decoder's own activation shapes (the
    # generator's last two stages for 128 phoneme ids: [1,256,71800] and
    # [1,128,430800] fp32), where the target of 70% of HBM peak applies.
    # InstanceNorm+affine is the graph's fused chain (statistics in numpy's
    # order: three reads and one write of x; its line counts the two
    # algorithmic passes).
    for C, T in ((256, 71800), (128, 430800)):
        nbytes = 4 * C * T
        nd = max(2, -(-ROTATE_BYTES // (2 * nbytes)))
        dx = B.replicate(D(r.normal(0, 1, (1, C, T)).astype(np.float32)), nd)
        do = [kk.DeviceTensor.empty((1, C, T)) for _ in range(nd)]
        dc = D(r.normal(0, 1, (1, C, 1)).astype(np.float32))
        da = D(r.uniform(0.5, 2, (1, C, 1)).astype(np.float32))
        dg = D((1 + 0.1 * r.normal(0, 1, (1, C, 1))).astype(np.float32))
        tag = f"1x{C}x{T}"
        copies[tag] = per_op(f"copy_{tag}", lambda i: B.call("kk_copy", do[i].desc(), dx[i].desc()),
                             2 * nbytes, sets=nd)
        vs_copy(per_op(f"add_{tag}", lambda i: B.call("kk_binary", opc["Add"], do[i].desc(),
                                                       dx[i].desc(), dc.desc()), 2 * nbytes + 4 * C,
                       sets=nd), tag)
        vs_copy(per_op(f"mul_{tag}", lambda i: B.call("kk_binary", opc["Mul"], do[i].desc(),
                                                       dx[i].desc(), dc.desc()), 2 * nbytes + 4 * C,
                       sets=nd), tag)
        vs_copy(per_op(f"leakyrelu_{tag}", lambda i: B.call("kk_unary", opc["LeakyRelu"], do[i].desc(),
                                                             dx[i].desc(), 0.2), 2 * nbytes, sets=nd), tag)
        vs_copy(per_op(f"snake_{tag}", lambda i: B.call("kk_snake", do[i].desc(), dx[i].desc(),
                                                         da.desc(), None), 2 * nbytes + 4 * C,
                       sets=nd), tag)
        vs_copy(per_op(f"instnorm_affine_{tag}", lambda i: B.call(
            "kk_instance_norm_scale_shift", do[i].desc(), dx[i].desc(), dg.desc(), dc.desc(), 1e-5, 0,
            0.0), 2 * nbytes + 8 * C, sets=nd, reps=10, eager=True), tag)
        del dx, do

    # dequant contractions (fp32 semantics; TFLOP/s against the fp32 peak)
    def gemm_case(name, m, k, n, wdt):
        a = B.replicate(D(r.normal(0, 1, (m, k)).astype(np.float32)), 4)
        if wdt == "i8":
            wq = D(r.integers(-127, 128, (k, n)).astype(np.int8))
            sc = D(np.array(r.uniform(1e-3, 1e-2), np.float32))
        else:
            wq = D(r.normal(0, 0.02, (k, n)).astype(np.float16))
            sc = None
        o = [kk.DeviceTensor.empty((m, n)) for _ in range(4)]
        # the constant weights packed once as the matrix cores' bf16 operands
        # (kk_gemm_pack); the per-call form (kk_gemm) converts them in the
        # kernel, also one launch
        pk = kk.ops.gemm_pack(wq)
        rec = per_op(name, lambda i: B.call("kk_gemm_packed", o[i].desc(), a[i].desc(), wq.desc(),
                                            pk.desc(), sc.desc() if sc else None, None, 1.0),
                     flops=2 * m * n * k, sets=4, mfma="bf16x3" if wdt == "i8" else "bf16x6")
        fu = lambda: [B.call("kk_gemm", o[i].desc(), a[i].desc(), wq.desc(), sc.desc() if sc else None,
                             None, 1.0) for _ in range(GRAPH_REPEAT) for i in range(4)]
        gid = B.graph(fu)
        rec["per_call_us"] = round(B.time_graphs([gid], 20) / (4 * GRAPH_REPEAT) * 1e3, 3)
        B.call("kk_graph_destroy", gid)

    gemm_case("gemm_i8_256x768x2048", 256, 768, 2048, "i8")
    gemm_case("gemm_i8_256x2048x768", 256, 2048, 768, "i8")
    gemm_case("gemm_f16_256x768x768", 256, 768, 768, "f16")

    def conv_case(name, cin, cout, k, L, pad, dil):
        x = B.replicate(D(r.normal(0, 1, (1, cin, L)).astype(np.float32)), 4)
        wq = D(r.integers(-127, 128, (cout, cin, k)).astype(np.int8))
        sc = D(np.array(0.005, np.float32))
        lout = L + 2 * pad - dil * (k - 1)
        o = [kk.DeviceTensor.empty((1, cout, lout)) for _ in range(4)]
        # the constant weights laid out once for the matrix cores, as the
        # graph does at load (kk_conv_pack); then one launch a call
        pk = kk.ops.conv_pack(wq, None, False, 1)
        rec = per_op(name, lambda i: B.call("kk_conv1d_packed", o[i].desc(), x[i].desc(), wq.desc(),
                                            pk.desc(), sc.desc(), None, None, 1, dil, pad, pad),
                     flops=2 * cout * cin * k * lout, sets=4, mfma="f16x2")
        # the per-call form (kk_conv1d): the layout made for every call
        fe = lambda i: B.call("kk_conv1d", o[i].desc(), x[i].desc(), wq.desc(), sc.desc(), None,
                              None, 1, dil, pad, pad, 1)
        rec["per_call_us"] = round(B.time_eager(fe, 4, 20) * 1e3, 3)
        rec["per_call_kernels"] = B.kernels_per_call(fe)

    conv_case("conv_i8_512x512_k3_L2400", 512, 512, 3, 2400, 1, 1)
    conv_case("conv_i8_256x256_k3_d1_L2400", 256, 256, 3, 2400, 1, 1)
    conv_case("conv_i8_256x256_k3_d3_L2400", 256, 256, 3, 2400, 3, 3)
    # ConvInteger on the int8 matrix cores at the 128-id decoder's largest
    # shape: uint8 x [1,128,431000], uint8 W [128,128,11], pad 5 (the int8
    # dense peak is 5.0 POP/s).
    L8 = 431000
    xq = B.replicate(D(r.integers(0, 256, (1, 128, L8)).astype(np.uint8)), 3)
    wq8 = D(r.integers(0, 256, (128, 128, 11)).astype(np.uint8))
    xz8, wz8 = D(np.array(119, np.uint8)), D(np.array(66, np.uint8))
    oq = [kk.DeviceTensor.empty((1, 128, L8), np.int32) for _ in range(3)]
    rec = per_op("conv_int8_128x128_k11_L431000", lambda i: B.call(
        "kk_conv_integer", oq[i].desc(), xq[i].desc(), wq8.desc(), xz8.desc(), wz8.desc(), 1, 1, 5,
        5, 1), flops=2 * 128 * 128 * 11 * L8, sets=3, reps=10, eager=True, mfma="i8")
    del xq, oq
    xt = B.replicate(D(r.normal(0, 1, (1, 512, 240)).astype(np.float32)), 4)
    wt = D(r.integers(-127, 128, (512, 256, 20)).astype(np.int8))
    sct = D(np.array(0.005, np.float32))
    ot = [kk.DeviceTensor.empty((1, 256, 2400)) for _ in range(4)]
    pkt = kk.ops.conv_pack(wt, None, True, 10)
    rec = per_op("convT_i8_512x256_k20_s10", lambda i: B.call(
        "kk_conv_transpose1d_packed", ot[i].desc(), xt[i].desc(), wt.desc(), pkt.desc(), sct.desc(),
        None, None, 10, 5, 5, 0), flops=2 * 512 * 256 * 2400 * 20 // 10, sets=4, mfma="f16x2")
    fe = lambda i: B.call("kk_conv_transpose1d", ot[i].desc(), xt[i].desc(), wt.desc(), sct.desc(),
                          None, None, 10, 1, 5, 5, 1, 0)
    rec["per_call_us"] = round(B.time_eager(fe, 4, 20) * 1e3, 3)
    rec["per_call_kernels"] = B.kernels_per_call(fe)

    # The decoder upsample stage as one chain of 13 ops: int8
    # ConvTranspose1d 512->256 (k20, s10, p5) on [1,512,240], snake, AdaIN
    # (style [1,128], Linear 128->512), then two residual blocks AdaIN ->
    # snake -> int8 Conv1d 256->256 k3 (dilation 1, then 3) -> AdaIN -> snake
    # -> int8 Conv1d k3 -> + input; per-tensor int8 scales.
    qt4 = D(r.integers(-127, 128, (512, 256, 20)).astype(np.int8))
    st4 = D(np.array(r.uniform(1e-3, 1e-2), np.float32))
    sty4 = D(r.normal(0, 0.1, (1, 128)).astype(np.float32))
    al4 = [D(r.uniform(0.5, 2, (1, 256, 1)).astype(np.float32)) for _ in range(5)]
    fc4 = [D(r.normal(0, 0.05, (128, 512)).astype(np.float32)) for _ in range(5)]
    cv4 = [(D(r.integers(-127, 128, (256, 256, 3)).astype(np.int8)),
            D(np.array(r.uniform(1e-3, 1e-2), np.float32))) for _ in range(4)]
    ops_ = kk.ops
    # the constant conv weights laid out once, as a graph does at load
    pq4 = ops_.conv_pack(qt4, None, True, 10)
    pcv4 = [ops_.conv_pack(q, None, False, 1) for q, _s in cv4]

    def stage4(i):
        h = ops_.conv_transpose1d(xt[i], qt4, None, (5, 5), 10, w_scale=st4, packed=pq4)
        h = ops_.adain(ops_.snake(h, al4[0]), sty4, fc4[0], None, 1e-5)
        for blk, dil in enumerate((1, 3)):
            y = ops_.snake(ops_.adain(h, sty4, fc4[1 + 2 * blk], None, 1e-5), al4[1 + 2 * blk])
            q, s = cv4[2 * blk]
            y = ops_.conv1d(y, q, None, (dil, dil), 1, dil, w_scale=s, packed=pcv4[2 * blk])
            y = ops_.snake(ops_.adain(y, sty4, fc4[2 + 2 * blk], None, 1e-5), al4[2 + 2 * blk])
            q, s = cv4[2 * blk + 1]
            y = ops_.conv1d(y, q, None, (1, 1), w_scale=s, packed=pcv4[2 * blk + 1])
            h = ops_.binary("Add", h, y)
        return h

    flops4 = 2 * 512 * 256 * 2400 * 20 // 10 + 4 * 2 * 256 * 256 * 3 * 2400
    # Recorded: the same 13 launches over buffers allocated beforehand, one
    # graph per rotating input set (device time, no host dispatch)
    hb = [[kk.DeviceTensor.empty((1, 256, 2400)) for _ in range(12)] for _ in range(4)]

    def stage4_rec(i):
        t = hb[i]
        c = lambda name, *a: B.call(name, *[v.desc() if isinstance(v, kk.DeviceTensor) else v
                                             for v in a])
        c("kk_conv_transpose1d_packed", t[0], xt[i], qt4, pq4, st4, None, None, 10, 5, 5, 0)
        c("kk_snake", t[1], t[0], al4[0], None)
        c("kk_adain", t[2], t[1], sty4, fc4[0], None, None, None, 1e-5)
        h, k = t[2], 3
        for blk, dil in enumerate((1, 3)):
            c("kk_adain", t[k], h, sty4, fc4[1 + 2 * blk], None, None, None, 1e-5)
            c("kk_snake", t[k + 1], t[k], al4[1 + 2 * blk], None)
            q, s = cv4[2 * blk]
            c("kk_conv1d_packed", t[k + 2], t[k + 1], q, pcv4[2 * blk], s, None, None, 1, dil, dil,
              dil)
            c("kk_adain", t[k], t[k + 2], sty4, fc4[2 + 2 * blk], None, None, None, 1e-5)
            c("kk_snake", t[k + 1], t[k], al4[2 + 2 * blk], None)
            q, s = cv4[2 * blk + 1]
            c("kk_conv1d_packed", t[k + 2], t[k + 1], q, pcv4[2 * blk + 1], s, None, None, 1, 1, 1,
              1)
            c("kk_binary", opc["Add"], t[k + 3], h, t[k + 2])
            h, k = t[k + 3], k + 4
        return h

    rec = per_op("decoder_upsample_stage_1x512x240", stage4_rec, flops=flops4, sets=4, reps=10)
    rec["ops"] = 13
    rec["workload"] = ("int8 ConvT 512->256 k20 s10 + snake + AdaIN, then 2 residual blocks "
                       "(AdaIN, snake, int8 Conv1d 256 k3 d1/d3, AdaIN, snake, Conv1d k3, Add); "
                       "weights packed at load")
    got = hb[0][10].numpy()  # the second block's sum
    want = stage4(0).numpy()  # the same chain through the op wrappers, eagerly
    if not np.array_equal(got, want):
        raise RuntimeError("bench: the recorded decoder stage differs from the eager one")
    rec["eager_us"] = round(B.time_eager(stage4, 4, 10) * 1e3, 3)

    # The output stage at the 128-id waveform's length (~2.15M samples): the
    # 1023-tap notch FIR (fp32 FMAs: 2 * 1023 flops per sample), the PCM16
    # conversion (4 B read, 2 B written per sample) and both in one pass.
    if not args.no_output_stage:
        output_stage_lines(kk, B, D, r, per_op)

    roofline = {
        "kernel": "instnorm_wide_kernel (AdaIN T=9600, style Linear fused)",
        "bound": "hbm",
        "achieved": dom["gbps"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(dom["gbps"] / HBM_PEAK_GBS, 4),
        "traffic": pmc_traffic("instnorm_wide_kernel"),
        "algorithmic_bytes_per_launch": BYTES["adain_t9600"],
        "avg_launch_us": dom["us"],
        "copy_same_size_gbps": cp["gbps"],
        "frac_of_copy": round(dom["gbps"] / cp["gbps"], 4),
    }
    return ms_per_step, nsets, ops_out, roofline


def run_graph(n_ids, reps):
    """Config 5: the full Kokoro-architecture graph (packed structure, seeded
    random learned weights) for `n_ids` phoneme ids.  Wall time runs from host
    input ids to the host waveform (uploads, the duration readback and the
    download included); the one-time weight upload and the text part's
    recording (on the token count's second run) are not timed: the timed
    runs replay the recorded text part and walk the rest."""
    kk = importlib.import_module("best-tts-godot_amd")
    kkg = importlib.import_module("best-tts-godot_amd.graph")
    g = kkg.load_graph()
    pg = kkg.PackedGraph(g, kkg.synth_weights(g, 0))
    ids, style, speed = kkg.synth_inputs(n_ids, 0)
    first = pg.run(ids, style, speed, keep=[2432])  # warm-up: fills the buffer pool
    frames = int(np.asarray(kk.to_host(pg.last_env["2432"])).sum())
    # two more: the first run of a token count finds its text part (the
    # nodes before the first read of device data), the second records it
    # as a HIP graph, which the timed runs replay
    for _ in range(2):
        pg.run(ids, style, speed)
    kk.sync()
    rec_end, rec_kernels, rec_arena, rec_error = pg.recorded(len(ids))
    walls = []
    d0 = kk.dispatch_count()
    for _ in range(reps):
        t0 = time.perf_counter()
        wav = pg.run(ids, style, speed)
        walls.append(time.perf_counter() - t0)
    dispatches = (kk.dispatch_count() - d0) // max(1, reps) + (rec_kernels or 0)
    wall = float(np.median(walls))
    audio = wav.size / 24000.0
    # The timed output is checked: finite, 600 samples per predicted frame,
    # not silent, and the same bits as the warm-up run.
    if not np.isfinite(wav).all():
        raise RuntimeError("kokoro graph: non-finite waveform")
    if wav.size != 600 * frames:
        raise RuntimeError(f"kokoro graph: {wav.size} samples for {frames} frames")
    if not float(np.sqrt(np.mean(np.square(wav, dtype=np.float64)))) > 1e-3:
        raise RuntimeError("kokoro graph: silent waveform")
    if not np.array_equal(wav, first):
        raise RuntimeError("kokoro graph: the timed run differs from the warm-up run")
    rec = {
        "audio_sec_per_wall_sec": round(audio / wall, 2),
        "wall_ms": round(wall * 1e3, 2),
        "wall_ms_runs": [round(w * 1e3, 2) for w in walls],
        "tokens_T": int(len(ids)),
        "frames_F": frames,
        "samples": int(wav.size),
        "audio_sec": round(audio, 3),
        "nodes": len(g["nodes"]),
        "launch_nodes": len(pg.nodes),
        "kernels_per_run": int(dispatches),
        "recorded_text_part": {"nodes": rec_end, "graph_kernels": rec_kernels,
                               "arena_bytes": rec_arena, "error": rec_error},
        "checked": "finite, 600 samples per frame, not silent, bit-identical across runs",
        "peak_pool_bytes": kk.pool_stats()[2],
        "workload": (f"full Kokoro-82M-architecture graph ({len(g['nodes'])} nodes, "
                     f"{len(pg.nodes)} after chain fusion; int8 GEMM/conv + fp16 weights, "
                     f"seeded random-init), {n_ids} phoneme ids U{{1..177}}, voice-pack row "
                     "style, speed 1.0"),
    }
    log(f"bench: kokoro graph {json.dumps(rec)}")
    return rec


def blas_info():
    """numpy's BLAS library, its version and thread count (threadpoolctl),
    and OPENBLAS_NUM_THREADS as set in the environment."""
    try:
        from threadpoolctl import threadpool_info
        libs = [f"{d.get('internal_api')} {d.get('version')} ({d.get('num_threads')} threads)"
                for d in threadpool_info() if d.get("user_api") == "blas"]
    except Exception:  # pragma: no cover - threadpoolctl is installed here
        libs = []
    return (f"BLAS: {', '.join(libs) or 'unknown'}; OPENBLAS_NUM_THREADS="
            f"{os.environ.get('OPENBLAS_NUM_THREADS', 'unset')}")


def run_graph_cpu(n_ids):
    """The oracle's whole-graph walk on a bounded sample (n_ids ids)."""
    from oracle import kpk_run
    kkg = importlib.import_module("best-tts-godot_amd.graph")
    g = kkg.load_graph()
    w = kkg.synth_weights(g, 0)
    ids, style, speed = kkg.synth_inputs(n_ids, 0)
    t0 = time.perf_counter()
    wav = kpk_run.run(g, w, ids, style, speed)
    wall = time.perf_counter() - t0
    return {
        "value": round(wav.size / 24000.0 / wall, 4),
        "unit": "audio-sec per wall-sec",
        "cores": len(os.sched_getaffinity(0)),
        "kind": "port",
        "sample": (f"numpy oracle whole-graph walk, {n_ids} ids ({len(ids)} tokens), "
                   f"{wav.size} samples in {wall:.1f} s; numpy ufuncs/einsum on 1 thread, "
                   f"BLAS matmuls on up to the visible cores; numpy {np.__version__}; "
                   f"{blas_info()}"),
    }


def run_cpu(seconds):
    """The numpy oracle on this host, single-threaded, over the same step."""
    from oracle import ref_ops as O
    try:
        from threadpoolctl import threadpool_limits
        limiter = threadpool_limits(limits=1)
    except Exception:  # pragma: no cover - threadpoolctl is installed here
        limiter = None
    h = reduction_inputs()

    def step():
        O.adain(h["x1200"], h["style"], h["w"], h["b"], 1e-5)
        O.adain(h["x9600"], h["style"], h["w"], h["b"], 1e-5)
        O.layernorm(h["ln"], h["g"], h["beta"], -1, 1e-12)
        O.softmax(h["sm"], -1)

    step()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    blas = blas_info()
    if limiter is not None:
        limiter.restore_original_limits()
    t = float(np.median(times))
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(STEP_BYTES / t / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"numpy oracle, full step (AdaIN T=1200 and T=9600 with Linear, LayerNorm, "
                   f"Softmax) x{len(times)} runs, median {t * 1e3:.1f} ms/step; 1 thread "
                   f"(threadpoolctl); {model or platform.processor()}; "
                   f"{len(os.sched_getaffinity(0))} cores visible; numpy {np.__version__}; "
                   f"{blas} (limited to 1 thread for this sample)"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--graph-ids", type=int, default=128)
    ap.add_argument("--graph-reps", type=int, default=5)
    ap.add_argument("--graph-cpu-ids", type=int, default=2)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-output-stage", action="store_true",
                    help="skip the FIR/PCM16 lines (rocprofv3's kernel trace crashes on them)")
    ap.add_argument("--graph-repeat", type=int, default=GRAPH_REPEAT,
                    help="calls of an op per rotating set in its timing graph (rocprofv3's "
                         "kernel trace crashes on graphs of 4)")
    args = ap.parse_args()
    globals()["GRAPH_REPEAT"] = max(1, args.graph_repeat)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the op layer shards by utterance with no collective)", file=sys.stderr)
        return 2
    ms_per_step, nsets, ops_out, roofline = run_gpu(args)
    graph = None
    if not args.no_graph:
        graph = run_graph(args.graph_ids, args.graph_reps)
        if not args.no_cpu:
            graph["cpu_baseline"] = run_graph_cpu(args.graph_cpu_ids)
    cpu = None if args.no_cpu else run_cpu(args.cpu_seconds)
    value = STEP_BYTES / (ms_per_step * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy draws; inputs resident in HBM)",
        "config": {
            "workload": ("reductions: AdaIN (InstanceNorm over T, eps 1e-5, style Linear "
                         "128->1024 fused) on [1,512,1200] and [1,512,9600]; LayerNorm(768, "
                         "eps 1e-12) on [1,256,768]; Softmax(last axis) on [1,12,256,256]"),
            "bytes_per_step": STEP_BYTES,
            "rotating_sets": nsets,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ops": ops_out,
        "kokoro_graph": graph,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
