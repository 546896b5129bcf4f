"""Fusion of the packed graph's node chains into single libkk launches.

The packed Kokoro graph spells three hot patterns as chains of small nodes,
each of which would otherwise read and write a full decoder activation
(up to [1, 128, 10^6] fp32):

  quantised conv tail   ConvInteger -> Add(int32 bias) -> Cast(float) -> Mul(scale)
                        (the Add is absent in a few blocks)
  InstanceNorm          ReduceMean -> Sub -> Mul(d, d) -> ReduceMean -> Add(eps)
                        -> Sqrt -> Div -> [Mul(scale)] -> [Add(shift)] -> [LeakyRelu]
  snake                 Mul(alpha, x) -> Sin -> Pow(2) -> Mul(recip) -> Add(x)
  InstanceNorm + snake  the two above back to back (the decoder's residual blocks)
  InstanceNorm [+ snake] -> Cast(float) -> DynamicQuantizeLinear   (the float result unstored)

`fuse` rewrites each chain whose intermediate tensors have no other reader
into one pseudo-node that `dispatch` runs as one kernel (the reference's
executor runs the chains node by node, executor.gd:733-843; the arithmetic
of every fused form follows the chain's own, see the kernels).  A fused node
takes the place of the chain's last node, where all of its inputs exist.
"""
from collections import defaultdict

import numpy as np


def _const(weights, name):
    """Host value of a constant weight, or None."""
    v = weights.get(name)
    if v is None:
        return None
    host = getattr(v, "host", v)
    return None if host is None else np.asarray(host)


def fuse(nodes, weights, protect=()):
    """nodes: [(op, ins, outs, attrs)] with string tensor names; weights:
    {name: value} (host arrays, or device tensors with a `.host` copy for
    small constants).  Tensors named in `protect` (the graph output and any
    tensor a caller wants to read) are never fused away.

    Returns (fused_nodes, groups): groups[k] lists the original node indices
    that fused node k replaces, in order."""
    protect = set(protect)
    readers = defaultdict(list)
    for i, (_op, ins, _outs, _at) in enumerate(nodes):
        for n in ins:
            if n:
                readers[n].append(i)

    def only_reader(name, want=None):
        """Index of the single node reading `name` (and, if given, of op
        `want`), or None."""
        r = readers.get(name, [])
        if name in protect or len(set(r)) != 1:
            return None
        j = r[0]
        if want is not None and nodes[j][0] != want:
            return None
        return j

    def other(ins, name):
        a = [n for n in ins if n != name]
        return a[0] if len(a) == 1 else None

    producer = {o: i for i, (_op, _ins, outs, _at) in enumerate(nodes) for o in outs if o}
    used = set()
    replace = {}  # index of the chain's last node -> (fused node, chain indices)

    def claim(chain, fused):
        if any(i in used for i in chain):
            return False
        used.update(chain)
        replace[chain[-1]] = (fused, chain)
        return True

    for i, (op, ins, outs, at) in enumerate(nodes):
        if i in used:
            continue
        if op == "ConvInteger" and int(at.get("group", 1)) == 1:
            _match_qconv(nodes, i, only_reader, other, claim)
        elif op == "MatMulInteger":
            _match_qmatmul(nodes, weights, producer, i, only_reader, other, claim)
        elif op == "ReduceMean":
            _match_instnorm(nodes, weights, i, only_reader, readers, protect, other, claim)
        elif op == "Sin":
            _match_snake(nodes, weights, i, only_reader, other, claim)

    out, groups = [], []
    for i, node in enumerate(nodes):
        if i in replace:
            fused, chain = replace[i]
            out.append(fused)
            groups.append(list(chain))
        elif i not in used:
            out.append(node)
            groups.append([i])
    out, groups = _merge_norm_snake(out, groups, protect)
    out, groups = _merge_norm_quant(out, groups, protect)
    out, groups = _merge_qconv_bias(out, groups, weights, protect)
    out, groups = _merge_qconv_add(out, groups, protect)
    return _link_conv_leaves(out), groups


def _link_conv_leaves(out):
    """An InstanceNormQuant whose x a quantised conv (with its bias
    quantisation folded in) produces takes that conv's leaf sums of x: the
    conv node gains a second output "<x>#leaves", the norm node a sixth
    input of that name (the dispatch forms the sums only for packed weights
    and rows long enough for the block-wise statistics, and the norm reads
    x again where there are none)."""
    producer = {}
    for k, (op, _ins, outs, at) in enumerate(out):
        if op == "QConvScaled" and at.get("bias_quant") and outs and outs[0]:
            producer[outs[0]] = k
    linked = list(out)
    for k, (op, ins, outs, at) in enumerate(out):
        if op != "InstanceNormQuant" or ins[0] not in producer:
            continue
        c = producer[ins[0]]
        name = f"{ins[0]}#leaves"
        c_op, c_ins, c_outs, c_at = linked[c]
        if len(c_outs) < 2:
            linked[c] = (c_op, c_ins, [c_outs[0], name], c_at)
        linked[k] = (op, list(ins[:5]) + [""] * (5 - len(ins[:5])) + [name], outs, at)
    return linked


def _merge_qconv_add(out, groups, protect):
    """An Add one of whose inputs is a quantised conv's output read by the
    Add alone (and not kept) takes the conv in (the decoder's residual sums):
    the conv's node, producing the Add's output, with the Add's other input
    appended (attribute "resid": its input index), placed where the Add was,
    so the residual already exists when it runs.  Whether the residual has the
    conv output's shape is known only when the node runs; dispatch adds it in
    the conv's epilogue then, else runs the Add after the conv."""
    readers = defaultdict(list)
    producer = {}
    for k, (_op, ins, outs, _at) in enumerate(out):
        for n in ins:
            if n:
                readers[n].append(k)
        for o in outs:
            if o:
                producer[o] = k
    takes = {}  # Add index -> (conv index, residual name)
    convs = set()
    for k, (op, ins, outs, _at) in enumerate(out):
        if op != "Add" or len(ins) != 2 or not ins[0] or not ins[1]:
            continue
        for side in (0, 1):
            name = ins[side]
            p = producer.get(name)
            if p is None or p in convs or out[p][0] != "QConvScaled" or "resid" in out[p][3]:
                continue
            if name in protect or readers.get(name) != [k] or len(out[p][2]) != 1:
                continue
            takes[k] = (p, ins[1 - side])
            convs.add(p)
            break
    if not takes:
        return out, groups
    new_out, new_groups = [], []
    for k, node in enumerate(out):
        if k in convs:
            continue
        if k in takes:
            p, resid = takes[k]
            c_op, c_ins, _c_outs, c_at = out[p]
            at = dict(c_at)
            at["resid"] = len(c_ins)
            new_out.append((c_op, list(c_ins) + [resid], list(node[2]), at))
            new_groups.append(list(groups[p]) + list(groups[k]))
        else:
            new_out.append(node)
            new_groups.append(groups[k])
    return new_out, new_groups


def _merge_qconv_bias(out, groups, weights, protect):
    """A quantised conv whose int32 bias the graph forms per call --
    scale = Mul(sa, sw); bias = Reshape(Cast(int32, Floor(Div(b, scale)))),
    every link read by the next alone and the scale by the Div and the conv
    alone -- takes those five nodes in: QConvScaled with bias_quant, inputs
    x, w, x_zp, w_zp, "", "", sa, sw, b.  Only where sa and sw are single
    values and b, a constant, has one value per output channel (the chain
    then broadcasts exactly per channel)."""
    readers = defaultdict(list)
    producer = {}
    for k, (_op, ins, outs, _at) in enumerate(out):
        for n in ins:
            if n:
                readers[n].append(k)
        for o in outs:
            if o:
                producer[o] = k

    def sole(name, k):
        return name not in protect and readers.get(name) == [k]

    def size(name):
        v = weights.get(name)
        return None if v is None else int(np.prod(getattr(v, "shape", ())))

    def single(name, depth=0):
        """One value: a one-element constant, or the scale output of a
        quantiser (DynamicQuantizeLinear, InstanceNormQuant), through Casts."""
        if size(name) is not None:
            return size(name) == 1
        p = producer.get(name)
        if p is None or depth > 4:
            return False
        p_op, p_ins, p_outs = out[p][0], out[p][1], out[p][2]
        if p_op == "Cast":
            return single(p_ins[0], depth + 1)
        return p_op in ("DynamicQuantizeLinear", "InstanceNormQuant") and \
            len(p_outs) > 1 and p_outs[1] == name

    takes = {}  # conv index -> indices of the five nodes it absorbs
    for k, (op, ins, outs, at) in enumerate(out):
        if op != "QConvScaled" or at.get("bias_quant") or len(ins) < 6 or not ins[4]:
            continue
        bias_i, scale = ins[4], ins[5]
        r = producer.get(bias_i)
        if r is None or out[r][0] != "Reshape" or not sole(bias_i, k):
            continue
        c = producer.get(out[r][1][0])
        if c is None or out[c][0] != "Cast" or int(out[c][3].get("to", 0)) != 6 or \
                not sole(out[r][1][0], r):
            continue
        f = producer.get(out[c][1][0])
        if f is None or out[f][0] != "Floor" or not sole(out[c][1][0], c):
            continue
        d = producer.get(out[f][1][0])
        if d is None or out[d][0] != "Div" or not sole(out[f][1][0], f) or \
                len(out[d][1]) != 2 or out[d][1][1] != scale:
            continue
        m = producer.get(scale)
        b = out[d][1][0]
        if m is None or out[m][0] != "Mul" or len(out[m][1]) != 2 or scale in protect or \
                sorted(readers.get(scale, [])) != sorted([d, k]):
            continue
        sa, sw = out[m][1]
        cout = getattr(weights.get(ins[1]), "shape", (None,))[0]
        if not (single(sa) and single(sw) and cout is not None and size(b) == cout):
            continue
        takes[k] = [m, d, f, c, r]
    if not takes:
        return out, groups
    dropped = {i for v in takes.values() for i in v}
    new_out, new_groups = [], []
    for k, node in enumerate(out):
        if k in dropped:
            continue
        if k in takes:
            m, d = takes[k][0], takes[k][1]
            op, ins, outs, at = node
            ins = list(ins[:4]) + ["", ""] + list(out[m][1]) + [out[d][1][0]]
            node = (op, ins, outs, dict(at, bias_quant=1))
            new_groups.append(sorted(sum((groups[i] for i in takes[k]), []) + groups[k]))
        else:
            new_groups.append(groups[k])
        new_out.append(node)
    return new_out, new_groups


def _merge_norm_quant(out, groups, protect):
    """An InstanceNorm chain (plain, with LeakyRelu or with the snake) whose
    result only a Cast(float) reads, and that Cast's result only a
    DynamicQuantizeLinear, becomes one InstanceNormQuant node at the
    quantiser's place: inputs x, scale, shift, alpha, recip; the quantiser's
    outputs (the float result is never stored)."""
    readers = defaultdict(list)
    for k, (_op, ins, _outs, _at) in enumerate(out):
        for n in ins:
            if n:
                readers[n].append(k)

    def sole(name):
        r = readers.get(name, [])
        return r[0] if name not in protect and len(set(r)) == 1 else None

    merged = {}  # quantiser index -> (norm index, cast index)
    for k, (op, ins, outs, at) in enumerate(out):
        if op not in ("InstanceNormScaleShift", "InstanceNormSnake"):
            continue
        c = sole(outs[0])
        if c is None or out[c][0] != "Cast" or int(out[c][3].get("to", 0)) != 1:
            continue
        q = sole(out[c][2][0])
        if q is None or out[q][0] != "DynamicQuantizeLinear" or out[q][1][0] != out[c][2][0]:
            continue
        merged[q] = (k, c)
    if not merged:
        return out, groups
    dropped = {i for pair in merged.values() for i in pair}
    new_out, new_groups = [], []
    for k, node in enumerate(out):
        if k in dropped:
            continue
        if k in merged:
            n, c = merged[k]
            n_op, n_ins, _n_outs, n_at = out[n]
            n_ins = list(n_ins) + [""] * (5 - len(n_ins))
            node = ("InstanceNormQuant", n_ins[:5], list(node[2]), dict(n_at))
            new_groups.append(groups[n] + groups[c] + groups[k])
        else:
            new_groups.append(groups[k])
        new_out.append(node)
    return new_out, new_groups


def _merge_norm_snake(out, groups, protect):
    """An InstanceNorm chain (without LeakyRelu) whose output only a snake
    chain reads becomes one InstanceNormSnake node, at the snake's place:
    inputs x, scale, shift, alpha, recip (the decoder's residual blocks:
    norm -> snake -> quantised conv)."""
    readers = defaultdict(list)
    for k, (_op, ins, _outs, _at) in enumerate(out):
        for n in ins:
            if n:
                readers[n].append(k)
    merged = {}  # snake index -> norm index
    for k, (op, ins, outs, at) in enumerate(out):
        if op != "InstanceNormScaleShift" or "leaky_alpha" in at:
            continue
        y = outs[0]
        r = readers.get(y, [])
        if y in protect or len(set(r)) != 1:
            continue
        j = r[0]
        s_op, s_ins, _s_outs, _s_at = out[j]
        if s_op == "Snake" and len(s_ins) == 3 and s_ins[0] == y and y not in s_ins[1:]:
            merged[j] = k
    if not merged:
        return out, groups
    dropped = set(merged.values())
    new_out, new_groups = [], []
    for k, node in enumerate(out):
        if k in dropped:
            continue
        if k in merged:
            n_op, n_ins, _n_outs, n_at = out[merged[k]]
            n_ins = list(n_ins) + [""] * (3 - len(n_ins))
            node = ("InstanceNormSnake", n_ins[:3] + list(node[1][1:3]), [node[2][0]], dict(n_at))
            new_groups.append(groups[merged[k]] + groups[k])
        else:
            new_groups.append(groups[k])
        new_out.append(node)
    return new_out, new_groups


def _match_qconv(nodes, i, only_reader, other, claim):
    op, ins, outs, at = nodes[i]
    acc = outs[0]
    j = only_reader(acc)
    if j is None:
        return
    chain = [i]
    bias = ""
    if nodes[j][0] == "Add":
        bias = other(nodes[j][1], acc)
        if bias is None:
            return
        chain.append(j)
        j = only_reader(nodes[j][2][0])
        if j is None:
            return
    if nodes[j][0] != "Cast" or int(nodes[j][3].get("to", 1)) not in (1, 10):
        return
    chain.append(j)
    k = only_reader(nodes[j][2][0], "Mul")
    if k is None:
        return
    scale = other(nodes[k][1], nodes[j][2][0])
    if scale is None:
        return
    chain.append(k)
    conv_ins = list(ins) + [""] * (4 - len(ins))
    fused = ("QConvScaled", conv_ins[:4] + [bias, scale], [nodes[k][2][0]], dict(at))
    claim(chain, fused)


def _match_qmatmul(nodes, weights, producer, i, only_reader, other, claim):
    """MatMulInteger -> Cast(float) -> Mul(scale) -> Add(bias), the Add only
    when its other operand is a float constant (the Linear's bias)."""
    op, ins, outs, at = nodes[i]
    j = only_reader(outs[0], "Cast")
    if j is None or int(nodes[j][3].get("to", 1)) not in (1, 10):
        return
    k = only_reader(nodes[j][2][0], "Mul")
    if k is None:
        return
    scale = other(nodes[k][1], nodes[j][2][0])
    if scale is None:
        return
    chain, bias, out = [i, j, k], "", nodes[k][2][0]
    a = only_reader(out, "Add")
    if a is not None:
        b = other(nodes[a][1], out)
        w = weights.get(b) if b is not None else None
        if w is not None and np.dtype(getattr(w, "dtype", np.float64)).kind == "f":
            chain.append(a)
            bias, out = b, nodes[a][2][0]
    mm_ins = list(ins) + [""] * (4 - len(ins))
    fused_ins, attrs = mm_ins[:4] + [scale, bias], {}
    # the scale formed by a Mul that only this chain reads: its two factors
    # go in instead (the epilogue forms the product, rounded once)
    m = producer.get(scale)
    if m is not None and nodes[m][0] == "Mul" and only_reader(scale) == k and \
            all(f for f in nodes[m][1]) and len(nodes[m][1]) == 2:
        chain.append(m)
        fused_ins = mm_ins[:4] + ["", bias] + list(nodes[m][1])
        attrs = {"scale_product": 1}
    claim(sorted(chain), ("QMatMulScaled", fused_ins, [out], attrs))


def _axes_of(nodes, weights, i):
    op, ins, outs, at = nodes[i]
    if len(ins) > 1 and ins[1]:
        a = _const(weights, ins[1])
        return None if a is None else [int(v) for v in a.reshape(-1)]
    a = at.get("axes")
    return None if a is None else [int(v) for v in np.asarray(a).reshape(-1)]


def _match_instnorm(nodes, weights, i, only_reader, readers, protect, other, claim):
    op, ins, outs, at = nodes[i]
    axes = _axes_of(nodes, weights, i)
    if axes not in ([2], [-1]) or not int(at.get("keepdims", 1)):
        return
    x, m1 = ins[0], outs[0]
    a = only_reader(m1, "Sub")
    if a is None or nodes[a][1] != [x, m1]:
        return
    d = nodes[a][2][0]
    rd = readers.get(d, [])
    if d in protect or len(rd) != 3:  # Mul reads it twice, Div once
        return
    sq_i = [r for r in rd if nodes[r][0] == "Mul" and nodes[r][1] == [d, d]]
    div_i = [r for r in rd if nodes[r][0] == "Div" and nodes[r][1][0] == d]
    if len(set(sq_i)) != 1 or len(div_i) != 1:
        return
    b, g = sq_i[0], div_i[0]
    c = only_reader(nodes[b][2][0], "ReduceMean")
    if c is None or nodes[c][1][0] != nodes[b][2][0] or _axes_of(nodes, weights, c) != axes:
        return
    if not int(nodes[c][3].get("keepdims", 1)):
        return
    e = only_reader(nodes[c][2][0], "Add")
    if e is None:
        return
    eps_name = other(nodes[e][1], nodes[c][2][0])
    eps = _const(weights, eps_name) if eps_name else None
    if eps is None or eps.size != 1:
        return
    f = only_reader(nodes[e][2][0], "Sqrt")
    if f is None or only_reader(nodes[f][2][0]) != g or nodes[g][1] != [d, nodes[f][2][0]]:
        return
    chain = [i, a, b, c, e, f, g]
    y = nodes[g][2][0]
    scale = shift = ""
    alpha = None
    k = only_reader(y, "Mul")
    if k is not None:
        s = other(nodes[k][1], y)
        if s is not None:
            scale, y = s, nodes[k][2][0]
            chain.append(k)
            k = only_reader(y, "Add")
            if k is not None:
                s = other(nodes[k][1], y)
                if s is not None:
                    shift, y = s, nodes[k][2][0]
                    chain.append(k)
                    k = only_reader(y, "LeakyRelu")
                    if k is not None:
                        alpha = float(nodes[k][3].get("alpha", 0.01))
                        y = nodes[k][2][0]
                        chain.append(k)
    attrs = {"epsilon": float(np.float32(eps.reshape(-1)[0]))}
    if alpha is not None:
        attrs["leaky_alpha"] = alpha
    claim(chain, ("InstanceNormScaleShift", [x, scale, shift], [y], attrs))


def _match_snake(nodes, weights, i, only_reader, other, claim):
    op, ins, outs, at = nodes[i]
    # Mul(alpha, x) feeding the Sin
    prods = [p for p, n in enumerate(nodes) if n[2] and n[2][0] == ins[0]]
    if len(prods) != 1:
        return
    p = prods[0]
    if nodes[p][0] != "Mul" or only_reader(ins[0]) != i:
        return
    m_ins = nodes[p][1]
    wts = [n for n in m_ins if n in weights]
    if len(wts) != 1 or len(m_ins) != 2:
        return
    alpha = wts[0]
    x = other(m_ins, alpha)
    if x is None:
        return
    q = only_reader(outs[0], "Pow")
    if q is None:
        return
    two = _const(weights, nodes[q][1][1]) if len(nodes[q][1]) > 1 else None
    if two is None or two.size != 1 or float(two.reshape(-1)[0]) != 2.0:
        return
    r = only_reader(nodes[q][2][0], "Mul")
    if r is None:
        return
    recip = other(nodes[r][1], nodes[q][2][0])
    if recip is None or recip not in weights:
        return
    s = only_reader(nodes[r][2][0], "Add")
    if s is None or sorted(nodes[s][1]) != sorted([x, nodes[r][2][0]]):
        return
    claim([p, i, q, r, s], ("Snake", [x, alpha, recip], [nodes[s][2][0]], {}))
