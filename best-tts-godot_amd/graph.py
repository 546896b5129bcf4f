"""Packed-graph runner: the Kokoro graph walked node by node through the
drop-in dispatch on the GPU.

The walk restates PackedModel.run (tools/kpk_runtime.py:52-81) with the GPU
executor's memory discipline (executor.gd:190-195, 270-280): every
intermediate tensor is dropped from `env` after its last use, which returns
its buffer to libkk's pool.

A model comes from a KPK1 file (`PackedGraph.from_kpk`, the format the
reference ships its model in, tools/pack_model.py:11-19) or from a graph
description and its weights.  The package carries the structure of the
Kokoro-82M graph (`data/kokoro_graph.json.gz`: nodes, ops, shapes, structural
constants and per-tensor statistics of the learned weights, extracted from
the reference's model.kpk); `synth_weights` draws seeded random learned
weights of the same dtype, shape and scale, which together give the full
Kokoro-82M-architecture graph with random-init weights (int8/uint8 for the
quantized contractions, fp16 elsewhere); `synth_model` packs the two.
"""
import collections
import ctypes
import gzip
import json
import os

import numpy as np

from . import _lib, audio, ops
from . import tensor as _tensor
from .dispatch import dispatch, to_device, to_host
from .fuse import fuse as fuse_chains
from .kpk import CODE_TO_NP, read_kpk
from .tensor import DeviceTensor, pool_stats

DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data")


def structure_path():
    """The packaged structure of the Kokoro-82M graph."""
    return os.path.join(DATA, "kokoro_graph.json.gz")


def load_graph(path=None):
    """The graph description at `path` (default: the packaged structure)."""
    with gzip.open(path or structure_path(), "rt") as f:
        return json.load(f)


# Three learned tensors of the synthetic model are not drawn at the trained
# tensors' statistics, so that it produces voiced excitation and an
# audio-range waveform:
#  * the pitch head (F0_proj) is a monotone 150 Hz voice: its quantised
#    weights all equal their zero point (so the conv's sum is exactly 0)
#    and its bias is 150 Hz.  Drawn at their statistics the weights lack
#    the trained head's structure and give |F0| < 2 Hz, below the sine
#    source's voiced threshold: the harmonic source is then a constant whose
#    STFT frames are all alike, and the generator's instance norms divide a
#    zero-padding step at the two ends by a near-zero spread -- a 10x edge
#    transient that sets every quantiser's range behind it.  A random head
#    at a voiced level does not do either, but its F0 carries the
#    predictor's quantisation noise (~1e-4 relative between two fp32
#    implementations), which the sine source integrates over 10^5 samples
#    and 9 harmonics into phase differences of radians; a constant head
#    leaves F0 equal to within one quantum of the bias (~2e-5 Hz);
#  * the generator's output projection (conv_post, whose first 11 channels
#    are log-magnitudes fed to Exp) is drawn at 1/20 of the trained std:
#    with random weights the activations reaching it are ~20x the trained
#    model's (|x| ~ 100 against ~5), which would put the log-magnitudes at
#    +-50 (exp ~ 1e21); scaled, they stay within +-2.5 and the waveform has
#    an RMS of ~0.25.
PITCH_WEIGHT = "encoder.predictor.F0_proj.weight_quantized"
PITCH_BIAS = ("encoder.predictor.F0_proj.bias", 150.0)
OUTPUT_HEAD = ("/decoder/decoder/generator/Mul_2_output_0", 1.0 / 20.0)


def _zero_point_of(graph, tid):
    """The constant weight zero point of the ConvInteger / MatMulInteger that
    reads weight tensor `tid` (input 3), or 0."""
    for op, ins, _outs, _at, _pl in graph["nodes"]:
        if graph["ops"][op] in ("ConvInteger", "MatMulInteger") and len(ins) > 1 and ins[1] == tid:
            if len(ins) > 3 and ins[3] >= 0 and "v" in graph["weights"].get(str(ins[3]), {}):
                return graph["weights"][str(ins[3])]["v"][0]
            return 0
    return 0


def synth_weights(graph, seed=0):
    """{tensor id: ndarray}: structural constants exact, learned tensors drawn
    from N(mean, std) of the original tensor, clipped to its [min, max] (and
    rounded for the integer types), one RNG stream per tensor id; the pitch
    head and the output head as stated above."""
    out = {}
    names = graph.get("tensors", [])
    for tid, w in graph["weights"].items():
        dt = CODE_TO_NP[w["d"]]
        shape = tuple(w["s"])
        name = names[int(tid)] if int(tid) < len(names) else ""
        if name == PITCH_BIAS[0]:
            out[int(tid)] = np.full(shape, PITCH_BIAS[1], dtype=dt)
            continue
        if name == PITCH_WEIGHT:
            out[int(tid)] = np.full(shape, _zero_point_of(graph, int(tid)), dtype=dt)
            continue
        if "v" in w:
            out[int(tid)] = np.array(w["v"], dtype=dt).reshape(shape)
            continue
        mean, std, lo, hi = w["stat"]
        if name == OUTPUT_HEAD[0]:
            mean, std, lo, hi = (v * OUTPUT_HEAD[1] for v in (mean, std, lo, hi))
        r = np.random.default_rng([int(seed), int(tid)])
        v = r.normal(mean, std, shape)
        if np.dtype(dt).kind in "iu":
            info = np.iinfo(dt)
            v = np.clip(np.rint(v), max(lo, info.min), min(hi, info.max))
        else:
            v = np.clip(v, lo, hi)
        out[int(tid)] = v.astype(dt)
    return out


def synth_inputs(n_ids=128, seed=0):
    """128 phoneme ids U{1..177} padded with 0 at both ends; a voice pack
    [510, 1, 256] ~ N(0, 0.1) indexed by length (row len(ids) - 3, as
    tools/voice_util.py:49-57 does for the padded ids); speed 1.0."""
    r = np.random.default_rng(seed)
    ids = np.concatenate([[0], r.integers(1, 178, n_ids), [0]]).astype(np.int64)
    pack = r.normal(0, 0.1, (510, 1, 256)).astype(np.float32)
    style = pack[min(max(len(ids) - 3, 0), 509)].reshape(1, 256)
    return ids, style, 1.0


def _decode_attrs(at):
    attrs = {}
    for k, v in (at or {}).items():
        if isinstance(v, dict) and "__t" in v:
            v = np.array(v["v"], dtype=CODE_TO_NP[v["__t"]]).reshape(v["s"])
        attrs[k] = v
    return attrs


class NonFiniteError(RuntimeError):
    """A strict run's first node with a non-finite float output: `node`
    (index in the walk), `op`, `output` (tensor name) and `inputs` (name,
    shape, dtype, (min, max)) of each of its inputs."""

    def __init__(self, msg, node, op, output, inputs):
        super().__init__(msg)
        self.node, self.op, self.output, self.inputs = node, op, output, inputs


class _TextPart:
    """The nodes a run walks before its first read of device data -- the
    text encoder, the predictors and the durations, whose shapes follow from
    the token count alone -- recorded for one token count as one HIP graph
    that owns its intermediates (kk_graph_begin_arena)."""

    __slots__ = ("end", "arena", "gid", "inputs", "env", "checks", "error")

    def __init__(self):
        self.end = None     # nodes [0, end) are recorded
        self.arena = 0      # arena bytes to record with
        self.gid = None     # the recorded graph
        self.inputs = None  # device input_ids, style, speed the graph reads
        self.env = None     # the tensors live after node end - 1
        self.checks = ()    # (node, axis, extent) of the Gathers indexed by input_ids
        self.error = None   # why this token count is walked without recording


class PackedGraph:
    """A packed graph with its weights resident on the device.

    With `fuse` (the default) the quantised-conv tails, InstanceNorm chains
    and snake chains run as single kernels; `groups[k]` lists the original
    node indices that node k stands for.  Tensors in `protect` stay
    readable after a run (they are never fused away).

    With `record` (the default) the part of a run that precedes its first
    read of device data is recorded as a HIP graph on the second run of a
    token count and replayed from the third on, from device copies of the
    inputs: the same kernels with the same arguments, without walking those
    nodes on the host.  The first run of a token count finds where that part
    ends; up to `RECORD_KEEP` token counts keep their graphs."""

    RECORD_KEEP = 4

    @classmethod
    def from_kpk(cls, path, fuse=True, protect=(), record=True):
        """The model in the KPK1 file at `path` (tools/kpk_runtime.py:27-50)."""
        desc, weights = read_kpk(path)
        return cls(desc, weights, fuse=fuse, protect=protect, record=record)

    def __init__(self, graph, weights, fuse=True, protect=(), record=True):
        self.record = record
        self._parts = collections.OrderedDict()  # token count -> _TextPart
        self.graph = graph
        self._notch = None  # the notch filter's taps on the device, made on first use
        self.ops = graph["ops"]
        nodes = [(self.ops[op], ["" if t < 0 else str(t) for t in ins],
                  ["" if t < 0 else str(t) for t in outs], _decode_attrs(at))
                 for op, ins, outs, at, _pl in graph["nodes"]]
        self.inputs = {k: str(v) for k, v in graph["inputs"].items()}
        self.output = str(graph["output"])
        # Weights: float data on the device once (fp16 widened to fp32 there,
        # except the fp16 weights that only Conv/ConvTranspose read, which
        # keep fp16 for the fp16 matrix-core convolutions), integer data
        # as-is; integer constants also stay on the host, where the
        # shape-domain nodes read them.
        conv_w, other = set(), set()
        for op, ins, _outs, _at in nodes:
            for k, name in enumerate(ins):
                (conv_w if op in ("Conv", "ConvTranspose") and k == 1 else other).add(name)
        conv_w -= other
        self.weights = {}
        for tid, arr in weights.items():
            arr = np.asarray(arr)
            if arr.dtype.kind in "iub" and arr.dtype.itemsize >= 4 or arr.dtype == np.bool_:
                self.weights[str(tid)] = arr
                continue
            if arr.dtype == np.float16 and str(tid) in conv_w:
                self.weights[str(tid)] = to_device(arr)
                continue
            if arr.dtype == np.float16:
                t = to_device(arr).astype(np.float32)
                host = arr.astype(np.float32)
            else:
                t = to_device(arr)
                host = arr
            if arr.size <= 16:
                t.host = host  # small constants are also read on the host
            self.weights[str(tid)] = t
        if fuse:
            keep = {self.output} | {str(p) for p in protect}
            self.nodes, self.groups = fuse_chains(nodes, self.weights, keep)
            self._pack_conv_weights()
        else:
            self.nodes, self.groups = nodes, [[i] for i in range(len(nodes))]
        # Last use of every non-weight tensor (executor.gd:190-195).
        self.last_use = {}
        for i, (_op, ins, _outs, _at) in enumerate(self.nodes):
            for name in ins:
                if name and name not in self.weights:
                    self.last_use[name] = i
        self.last_use.pop(self.output, None)
        self.frees = [[] for _ in self.nodes]  # names whose last use is node i
        for name, i in self.last_use.items():
            self.frees[i].append(name)

    def _pack_conv_weights(self):
        """Each fused quantised Linear (QMatMulScaled) with a constant 2-D B
        gets B packed once (ops.matmul_integer_pack), under
        "<B>#i8packed", named in its node's attribute "packed".  Each
        quantised conv with its bias quantisation folded in whose
        weight and weight zero point are constants gets its weights packed
        once (ops.conv_integer_pack), under "<weight>#packed"; its node names
        that in attribute "packed" and skips the per-call re-layout.  So does
        each Conv / ConvTranspose with a constant fp16 weight that the fp16
        matrix cores take (group 1, a transposed one with dilation 1, at
        most 8 taps a row: ops.conv_pack)."""
        packs = {}
        for k, (op, ins, outs, at) in enumerate(self.nodes):
            if op in ("Conv", "ConvTranspose"):
                self._pack_fp16_conv(k, op, ins, outs, at, packs)
                continue
            if op == "QMatMulScaled":
                # a constant 2-D B: packed once for the int8 matrix cores
                # (ops.matmul_integer_pack)
                bt = self.weights.get(ins[1])
                if isinstance(bt, DeviceTensor) and bt.ndim == 2 and bt.dtype in (np.int8, np.uint8):
                    key = (ins[1], "i8")
                    if key not in packs:
                        packs[key] = f"{ins[1]}#i8packed"
                        self.weights[packs[key]] = ops.matmul_integer_pack(bt)
                    self.nodes[k] = (op, ins, outs, dict(at, packed=packs[key]))
                continue
            if op != "QConvScaled" or not at.get("bias_quant"):
                continue
            w, wz = ins[1], ins[3]
            if w not in self.weights or (wz and wz not in self.weights):
                continue
            if wz and not isinstance(self.weights[wz], DeviceTensor):
                # an int32 zero point is kept on the host (integer constants
                # of 4 bytes or more are); the pack and every call read one
                # device copy of it (libkk checks that a call passes the
                # weight and zero-point tensors its pack was made from)
                dev = f"{wz}#dev"
                if dev not in self.weights:
                    self.weights[dev] = to_device(self.weights[wz])
                ins = list(ins)
                ins[3] = wz = dev
            key = (w, wz)
            if key not in packs:
                packs[key] = f"{w}#{wz}#packed"
                self.weights[packs[key]] = ops.conv_integer_pack(
                    self.weights[w], self.weights[wz] if wz else None)
            self.nodes[k] = (op, ins, outs, dict(at, packed=packs[key]))

    def _pack_fp16_conv(self, k, op, ins, outs, at, packs):
        w = ins[1] if len(ins) > 1 else ""
        wt = self.weights.get(w)
        if not isinstance(wt, DeviceTensor) or wt.dtype != np.float16 or wt.ndim != 3:
            return
        tr = op == "ConvTranspose"
        stride = int(at.get("strides", [1])[0])
        if int(at.get("group", 1)) != 1 or (tr and int(at.get("dilations", [1])[0]) != 1):
            return
        taps = -(-wt.shape[2] // stride) if tr else wt.shape[2]
        if taps > 8:
            return
        key = (w, tr, stride if tr else 1)
        if key not in packs:
            packs[key] = f"{w}#{'t' if tr else 'c'}{key[2]}#packed"
            self.weights[packs[key]] = ops.conv_pack(wt, None, tr, key[2])
        self.nodes[k] = (op, ins, outs, dict(at, packed=packs[key]))

    def _check_finite(self, i, env):
        """Strict mode (ref_runtime.py:404-418): raises at the first float
        output of node i that holds a NaN or an infinity, naming the node
        (and the original nodes it stands for) with the shape, dtype and
        value range of each of its inputs."""
        op, ins, outs, _at = self.nodes[i]
        for o in outs:
            v = env.get(o) if o else None
            if v is None or np.dtype(v.dtype).kind != "f" or not int(np.prod(v.shape)):
                continue
            host = np.asarray(to_host(v))
            if np.isfinite(host).all():
                continue
            bad = int((~np.isfinite(host)).sum())
            described = []
            for name in ins:
                if not name or name not in env:
                    continue
                a = np.asarray(to_host(env[name]))
                rng = None
                if a.dtype.kind in "fiu" and a.size:
                    af = a.astype(np.float64)
                    rng = (float(np.nanmin(af)), float(np.nanmax(af))) if not np.isnan(af).all() \
                        else (float("nan"), float("nan"))
                described.append((name, tuple(a.shape), str(a.dtype), rng))
            raise NonFiniteError(
                f"non-finite output at node {i} {op} (original nodes {self.groups[i]}) -> {o} "
                f"{tuple(v.shape)}: {bad} non-finite values\n  inputs: {described}",
                node=i, op=op, output=o, inputs=described)

    def _walk(self, env, lo, hi, keep, strict, probe=None):
        """Runs nodes [lo, hi) on `env`, dropping each tensor after its last
        use.  With `probe` (a _TextPart of this token count), also finds the
        first node that reads device data and the most pool memory the nodes
        before it hold at once."""
        frees = self.frees
        base = peak = pool_stats()[0] if probe is not None else 0
        for i in range(lo, hi):
            op, ins, outs, at = self.nodes[i]
            if probe is not None:
                seen = _tensor._state["downloads"]
            try:
                dispatch(op, ins, outs, at, env)
            except Exception as exc:
                raise RuntimeError(f"node {i} {op}: {exc}") from exc
            if probe is not None:
                if _tensor._state["downloads"] != seen:
                    self._measured(probe, i, peak - base)
                    probe = None
                else:
                    peak = max(peak, pool_stats()[0])
            if strict:
                self._check_finite(i, env)
            for name in frees[i]:
                if name not in keep:
                    env.pop(name, None)
        if probe is not None:
            self._measured(probe, hi, peak - base)

    # ------------------------------------------------ recorded text parts
    def _part(self, n_ids):
        part = self._parts.get(n_ids)
        if part is not None:
            self._parts.move_to_end(n_ids)
            return part
        while len(self._parts) >= self.RECORD_KEEP:
            self._drop(self._parts.popitem(last=False)[1])
        part = self._parts[n_ids] = _TextPart()
        return part

    def _measured(self, part, end, need):
        """Nodes [0, end) read no device data and held at most `need` bytes
        of the pool at once: record them in an arena of three times that (its
        buckets are not shared between sizes) and some slack.  The Gathers
        that index a weight with input_ids are checked on the host, as the
        walk checks host indices (a recorded gather clamps them)."""
        part.end = end
        part.arena = 3 * int(need) + (16 << 20)
        if end == 0:
            part.error = "the first node reads device data"
            return
        name = self.inputs["input_ids"]
        checks = []
        for i in range(end):
            op, ins, _outs, at = self.nodes[i]
            if name not in ins:
                continue
            data = self.weights.get(ins[0]) if op == "Gather" and ins.index(name) == 1 else None
            if op == "Shape":
                continue
            if data is None:
                part.error = f"node {i} {op} reads input_ids"
                return
            axis = int(at.get("axis", 0)) % len(data.shape)
            checks.append((i, axis, int(data.shape[axis])))
        part.checks = tuple(checks)

    def _record(self, part, env, ids, style, speed):
        """Walks nodes [0, part.end) into a graph with device inputs and
        launches it.  Returns part.end, or None when the walk could not be
        recorded (part.error says why; `env` then holds the weights only)."""
        names = self.inputs
        inputs = (DeviceTensor.from_numpy(ids), to_device(style), to_device(speed))
        env[names["input_ids"]], env[names["style"]], env[names["speed"]] = inputs
        failed = None
        _lib.call("kk_graph_begin_arena", part.arena)
        try:
            self._walk(env, 0, part.end, set(), False)
        except Exception as exc:  # recorded nothing that will run: walk it instead
            failed = f"{type(exc).__name__}: {exc}"
        gid = ctypes.c_int(-1)
        if failed is None:
            try:
                _lib.call("kk_graph_end", ctypes.byref(gid))
            except Exception as exc:
                failed = f"{type(exc).__name__}: {exc}"
        if failed is not None:
            # nothing may refer to the arena's blocks when it is released
            env.clear()
            env.update(self.weights)
            _lib.call("kk_graph_abort")
            part.error = failed
            return None
        part.gid = gid.value
        part.inputs = inputs
        part.env = {k: v for k, v in env.items() if k not in self.weights}
        _lib.call("kk_graph_launch", part.gid)
        return part.end

    def _replay(self, part, env, ids, style, speed):
        for i, axis, n in part.checks:
            if ids.size and (int(ids.min()) < -n or int(ids.max()) >= n):
                raise RuntimeError(
                    f"node {i} Gather: index out of bounds for axis {axis} with size {n}")
        for t, a in zip(part.inputs, (ids, style, speed)):
            _lib.call("kk_upload", ctypes.c_void_p(t.ptr), a.ctypes.data_as(ctypes.c_void_p),
                      a.nbytes)
        _lib.call("kk_graph_launch", part.gid)
        env.update(part.env)
        return part.end

    def _drop(self, part):
        gid, part.gid = part.gid, None
        part.env = part.inputs = None  # (before the graph's arena goes)
        if gid is not None and _lib._lib is not None:
            _lib.call("kk_graph_destroy", gid)

    def release_recordings(self):
        """Destroys the recorded text parts and frees their memory."""
        while self._parts:
            self._drop(self._parts.popitem()[1])

    def recorded(self, n_ids):
        """(recorded nodes, graph kernel nodes, arena bytes, error) of the
        text part for `n_ids` token ids, or None before its first run."""
        part = self._parts.get(n_ids)
        if part is None:
            return None
        kernels = None
        if part.gid is not None:
            n = ctypes.c_int64(0)
            _lib.call("kk_graph_nodes", part.gid, ctypes.byref(n))
            kernels = n.value
        return part.end, kernels, part.arena, part.error

    def __del__(self):
        try:
            self.release_recordings()
        except Exception:  # interpreter shutdown: the process frees it
            pass

    def run(self, input_ids, style, speed=1.0, keep=(), pcm16=False, notch=True, gain=1.0,
            strict=False, max_nodes=None, start=0, inject=None):
        """Returns the waveform on the host: float32 samples, or with
        `pcm16` the 16-bit PCM samples (int16) the reference's output stage
        makes of them on the device (audio.gd:59-106), through the notch
        filter first unless `notch` is false.

        Debugging aids: `strict` stops at the first node whose float output
        is not finite and raises NonFiniteError naming it and its inputs'
        ranges (ref_runtime.py:378-418; every float output is read back, so
        it is slow); `max_nodes` runs only the first that many nodes of the
        walk (executor.gd:67-72, 306-307) and returns None when the output
        was not reached -- `keep` names the tensors to look at then, in
        `last_env`; `start` skips the walk's first nodes, whose outputs the
        rest reads from `inject` ({tensor id: array}, floats placed on the
        device), to run a part of the graph from given values."""
        ids = np.ascontiguousarray(np.asarray(input_ids, np.int64).reshape(1, -1))
        style = np.ascontiguousarray(np.asarray(style, np.float32).reshape(1, 256))
        speed = np.asarray([speed], np.float32)
        keep = {str(k) for k in keep}
        limit = len(self.nodes) if max_nodes is None or max_nodes < 0 else min(max_nodes, len(self.nodes))
        part = None
        if self.record and start == 0 and not inject and not keep and not strict \
                and limit == len(self.nodes):
            part = self._part(ids.shape[1])
        env = dict(self.weights)
        first = None
        if part is not None and part.gid is not None:
            first = self._replay(part, env, ids, style, speed)
        elif part is not None and part.end is not None and part.error is None:
            first = self._record(part, env, ids, style, speed)
        if first is None:
            env[self.inputs["input_ids"]] = ids
            env[self.inputs["style"]] = to_device(style)
            env[self.inputs["speed"]] = to_device(speed)
            for name, v in (inject or {}).items():
                v = np.asarray(v)
                env[str(name)] = to_device(v) if v.dtype.kind == "f" else v
            first = start
        probe = part if part is not None and part.end is None else None
        self._walk(env, first, limit, keep, strict, probe)
        self.last_env = {k: env[k] for k in keep if k in env}
        if self.output not in env:
            return None
        out = env[self.output]
        if pcm16:
            taps = None
            if notch:
                if self._notch is None:
                    self._notch = to_device(audio.notch_taps())
                taps = self._notch
            return to_host(audio.to_pcm16(out, taps, gain)).view("<i2")
        return to_host(out)


def synth_model(graph=None, seed=0):
    """(description, {tensor id: ndarray}) of the Kokoro-82M-architecture
    graph with seeded random learned weights, ready for `kpk.write_kpk`."""
    graph = graph if graph is not None else load_graph()
    desc = {k: v for k, v in graph.items() if k not in ("source", "weights")}
    return desc, synth_weights(graph, seed)


__all__ = ["load_graph", "structure_path", "synth_weights", "synth_model", "synth_inputs",
           "PackedGraph", "NonFiniteError", "DeviceTensor"]
