"""Replays a prepared plan of the host framework on the CPU oracle.

TEST INFRASTRUCTURE ONLY. Given the active node list of a Session (after
QDQ fusion and layout assignment) and the Graph it came from, every node is
executed with the oracle's restatement of the reference operator, on arrays
kept in the same physical layout as the device tensors (NHWC when the plan
says so), so any intermediate tensor can be compared bit for bit.
"""
from __future__ import annotations

import numpy as np

from . import pyoracle as O


def _nchw_to_phys(a, nhwc):
    return a.transpose(0, 2, 3, 1).copy() if nhwc and a.ndim == 4 else a


def _erf(x):
    from scipy.special import erf
    return erf(x)


def run_plan(plan, graph, feeds: dict, fmt_of, stop_after=None, source=None, skip_ops=(), keep_chain=False):
    """plan: Session.plan(); fmt_of(name) -> 0/1 layout of a tensor.
    Returns {tensor name: physical numpy array} of every produced tensor
    (keep_chain: also the tensors inside fused chains, e.g. the uint8 output
    of a QLinearMatMul whose dequantize chain was fused into it).

    source: optional callable name -> array. When given, every node reads its
    non-constant inputs through it (e.g. the device's own tensors), so each
    node is checked on exactly the inputs the device saw and fp32 rounding
    differences do not propagate. Nodes whose op is in skip_ops are not run
    (their outputs must then come from source)."""
    init = graph.initializers
    env = {}
    chain_env = {}   # tensors inside a fused chain (they exist only here)
    for k, v in feeds.items():
        env[k] = v

    def val(name):
        if name in init:
            return init[name]
        if name in chain_env:
            return chain_env[name]
        if source is not None and name not in feeds:
            return source(name)
        return env[name]

    def scal(name, default=0):
        if not name:
            return default
        return val(name).reshape(-1)[0]

    def exec_node(nd):
        op, ins, outs = nd["op"], nd["inputs"], nd["outputs"]
        extra = {}
        if op == "QuantizeLinear":
            zdt = init[ins[2]].dtype if len(ins) > 2 and ins[2] else np.uint8
            y = O.quantize_linear(val(ins[0]), float(scal(ins[1])), int(scal(ins[2])), zdt)
        elif op == "DequantizeLinear":
            y = O.dequantize_linear(val(ins[0]), float(scal(ins[1])), int(scal(ins[2])))
        elif op == "DynamicQuantizeLinear":
            y, ys, yz = O.dynamic_quantize_linear(val(ins[0]))
            extra = {outs[1]: np.array(ys, np.float32), outs[2]: np.array(yz, np.uint8)}
        elif op in ("Add", "Mul", "Sub", "Div"):
            a_, b_ = val(ins[0]).astype(np.float32), val(ins[1]).astype(np.float32)
            y = {"Add": np.add, "Mul": np.multiply, "Sub": np.subtract, "Div": np.divide}[op](a_, b_)
            y = y.astype(np.float32)
        elif op == "Softmax":
            x = val(ins[0]).astype(np.float64)
            e = np.exp(x - x.max(axis=-1, keepdims=True))
            y = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
        elif op == "LayerNormalization":
            a = graph.node_by_name(nd["name"]).attrs
            x = val(ins[0]).astype(np.float64)
            mean = x.mean(axis=-1, keepdims=True)
            var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
            yv = (x - mean) / np.sqrt(var + a.get("epsilon", 1e-5)) * val(ins[1]).astype(np.float64)
            if len(ins) > 2 and ins[2]:
                yv = yv + val(ins[2]).astype(np.float64)
            y = yv.astype(np.float32)
        elif op == "Gelu":
            x = val(ins[0]).astype(np.float64)
            y = (0.5 * x * (1.0 + _erf(x / np.sqrt(2.0)))).astype(np.float32)
        elif op == "MatMulInteger":
            # MatMulInteger.cpp:11-150: exact int32 sum of (a - a_zp)(b - b_zp)
            a_zp = int(scal(ins[2])) if len(ins) > 2 and ins[2] else 0
            b_zp = int(scal(ins[3])) if len(ins) > 3 and ins[3] else 0
            y = O.matmul_integer(val(ins[0]), val(ins[1]), a_zp, b_zp)
        elif op == "Cast":
            # Cast.cpp (Cast_array): (float)x, int32 rounding to nearest even
            y = val(ins[0]).astype(np.float32)
        elif op == "HardSwish":
            y = O.hardswish(val(ins[0]), post_op=bool(nd.get("post_op")))
        elif op in ("Relu", "Clip"):
            lo, hi = (0.0, np.inf) if op == "Relu" else (
                float(scal(ins[1], -np.inf)) if len(ins) > 1 else -np.inf,
                float(scal(ins[2], np.inf)) if len(ins) > 2 else np.inf)
            y = np.minimum(np.maximum(val(ins[0]).astype(np.float32), np.float32(lo)), np.float32(hi))
        elif op == "Transpose":
            perm = graph.node_by_name(nd["name"]).attrs.get("perm")
            y = np.ascontiguousarray(np.transpose(val(ins[0]), perm))
        elif op == "MultiHeadAttention":
            # com.microsoft MultiHeadAttention (MultiHeadAttention.cpp), created
            # by the host's attention fusion in place of the Softmax node of
            # the same name: scale from the Mul before it, heads from q's Reshape
            sm = graph.node_by_name(nd["name"])
            mul = next(g_ for g_ in graph.nodes if sm.inputs[0] in g_.outputs)
            cname = next(t for t in mul.inputs if t in init)
            scale = float(init[cname].reshape(-1)[0])
            rs = next(g_ for g_ in graph.nodes if g_.op == "Reshape" and g_.inputs[0] == ins[0])
            nh = int(init[rs.inputs[1]][2])
            q, k, v = (val(t).astype(np.float64) for t in ins[:3])
            B, S, Hd = q.shape
            hd = Hd // nh
            split = lambda t: t.reshape(B, S, nh, hd).transpose(0, 2, 1, 3)
            sc = np.matmul(split(q), split(k).transpose(0, 1, 3, 2)) * scale
            e = np.exp(sc - sc.max(axis=-1, keepdims=True))
            p_ = e / e.sum(axis=-1, keepdims=True)
            y = np.matmul(p_, split(v)).transpose(0, 2, 1, 3).reshape(B, S, Hd).astype(np.float32)
        elif op == "MatMul":
            y = np.matmul(val(ins[0]).astype(np.float64), val(ins[1]).astype(np.float64)).astype(np.float32)
        elif op == "QLinearConv" and val(ins[0]).ndim == 3:
            # 3-D tensors: exec_typed (RQ-S), NCW only
            a = graph.node_by_name(nd["name"]).attrs
            x = val(ins[0])
            w = init[ins[3]]
            pads = a.get("pads", [0, 0])
            cv = O.Conv1d(x.shape[0], x.shape[1], x.shape[2], w.shape[0], w.shape[2], group=a.get("group", 1),
                          stride=a.get("strides", [1])[0], dil=a.get("dilations", [1])[0], pads=(pads[0], pads[1]),
                          act_dtype=x.dtype.type, x_scale=float(scal(ins[1])), x_zp=int(scal(ins[2])),
                          w_scale=init[ins[4]], w_zp=init[ins[5]] if ins[5] else (),
                          y_scale=float(scal(ins[6])), y_zp=int(scal(ins[7])),
                          bias=init[ins[8]] if len(ins) > 8 and ins[8] else None)
            y, br = cv.run(x, w)
            nd["oracle_branch"] = br
        elif op == "QLinearConv":
            src = graph.node_by_name(nd["name"])
            a = src.attrs
            x = val(ins[0])
            w = init[ins[3]]
            x_nhwc, y_nhwc = fmt_of(ins[0]), fmt_of(outs[0])
            N = x.shape[0]
            Cc, H, W = (x.shape[3], x.shape[1], x.shape[2]) if x_nhwc else x.shape[1:]
            k = a.get("kernel_shape", list(w.shape[2:]))
            cv = O.Conv(N, Cc, H, W, w.shape[0], k[0], k[1], group=a.get("group", 1),
                        stride=tuple(a.get("strides", [1, 1])), dil=tuple(a.get("dilations", [1, 1])),
                        pads=tuple(a.get("pads", [0, 0, 0, 0])), x_nhwc=x_nhwc, y_nhwc=y_nhwc,
                        post_fn=nd["post_fn"], act_dtype=x.dtype.type,
                        x_scale=float(scal(ins[1])), x_zp=int(scal(ins[2])),
                        w_scale=init[ins[4]], w_zp=init[ins[5]] if ins[5] else (),
                        y_scale=float(scal(ins[6])), y_zp=int(scal(ins[7])),
                        bias=init[ins[8]] if len(ins) > 8 and ins[8] else None)
            y, br = cv.run(x, w)
            nd["oracle_branch"] = br
            fa = nd.get("fused_add")
            if fa:
                # conv + QLinearAdd in one kernel: the conv result is the add
                # operand that is not `other`, then the add runs as planned
                ai = fa["inputs"]
                chain_env[ai[3] if ai[0] == fa["other"] else ai[0]] = y
                y = O.qlinear_add(0, val(ai[0]), val(ai[3]), float(scal(ai[1])), int(scal(ai[2])),
                                  float(scal(ai[4])), int(scal(ai[5])), float(scal(ai[6])),
                                  int(scal(ai[7])))
        elif op == "QLinearMatMul":
            y = O.qlinear_matmul(val(ins[0]), np.float32(scal(ins[1])), int(scal(ins[2])),
                                 init[ins[3]], float(scal(ins[4])), int(scal(ins[5])),
                                 float(scal(ins[6])), int(scal(ins[7])), init[ins[7]].dtype)
        elif op == "QLinearAdd":
            a_, b_ = val(ins[0]), val(ins[3])
            if a_.shape != b_.shape:
                raise NotImplementedError("broadcast QLinearAdd in the plan replay")
            y = O.qlinear_add(0, a_, b_, float(scal(ins[1])), int(scal(ins[2])),
                              float(scal(ins[4])), int(scal(ins[5])), float(scal(ins[6])),
                              int(scal(ins[7])))
        elif op == "QLinearMul":
            a_, b_ = val(ins[0]), val(ins[3])
            args = (float(scal(ins[1])), int(scal(ins[2])), float(scal(ins[4])), int(scal(ins[5])),
                    float(scal(ins[6])), int(scal(ins[7])))
            if a_.shape == b_.shape:
                y = O.qlinear_mul(0, a_, b_, *args)
            elif a_.size == 1:
                y = O.qlinear_mul(2, a_, b_, *args)
            elif b_.size == 1:
                y = O.qlinear_mul(1, a_, b_, *args)
            else:
                # per channel: the full operand first, with its own scale / zero point
                full_is_a = a_.size >= b_.size
                nhwc = fmt_of(ins[0] if full_is_a else ins[3])
                full, ch = (a_, b_) if full_is_a else (b_, a_)
                C = full.shape[3] if nhwc else full.shape[1]
                HW = full.size // (full.shape[0] * C)
                fs, fz, cs_, cz = (args[0], args[1], args[2], args[3]) if full_is_a else \
                    (args[2], args[3], args[0], args[1])
                y = O.qlinear_mul(3, full, ch.reshape(-1), fs, fz, cs_, cz, args[4], args[5], C=C, HW=HW,
                                  y_nhwc=nhwc)
        elif op == "QLinearGlobalAveragePool":
            x = val(ins[0])
            nhwc = fmt_of(ins[0])
            y = O.qlinear_global_avgpool(x, float(scal(ins[1])), int(scal(ins[2])), float(scal(ins[3])),
                                         int(scal(ins[4])), nhwc=nhwc)
            sp = [1] * (x.ndim - 2)
            y = y.reshape((y.shape[0], *sp, y.shape[1]) if nhwc else (y.shape[0], y.shape[1], *sp))
        elif op == "QLinearAveragePool":
            a = graph.node_by_name(nd["name"]).attrs
            x = val(ins[0])
            nhwc = fmt_of(ins[0])
            k, st = a["kernel_shape"], a.get("strides", [1, 1])
            p_ = list(a.get("pads", [0, 0, 0, 0])) + [0] * 4
            H, W = (x.shape[1], x.shape[2]) if nhwc else (x.shape[2], x.shape[3])
            if a.get("ceil_mode", 0):
                oH = int(np.ceil(np.float32(H + p_[0] + p_[2] - k[0]) / np.float32(st[0]) + 1))
                oW = int(np.ceil(np.float32(W + p_[1] + p_[3] - k[1]) / np.float32(st[1]) + 1))
            else:
                oH = (H + p_[0] + p_[2] - k[0]) // st[0] + 1
                oW = (W + p_[1] + p_[3] - k[1]) // st[1] + 1
            y = O.qlinear_avgpool(x, k, st, (p_[0], p_[1]), oH, oW, float(scal(ins[1])), int(scal(ins[2])),
                                  float(scal(ins[3])), int(scal(ins[4])), nhwc=nhwc)
        elif op == "QLinearConcat":
            a = graph.node_by_name(nd["name"]).attrs
            xs = [val(ins[2 + 3 * i]) for i in range((len(ins) - 2) // 3)]
            nhwc = fmt_of(ins[2])
            nd_ = xs[0].ndim
            ax = a.get("axis", 0) % nd_
            if nhwc:
                outer = xs[0].shape[0] * xs[0].shape[1] * xs[0].shape[2]
                counts = [x.shape[3] for x in xs]
            else:
                outer = int(np.prod(xs[0].shape[:ax]))
                counts = [int(np.prod(x.shape[ax:])) for x in xs]
            y = O.qlinear_concat([x.reshape(-1) for x in xs], counts, outer,
                                 [float(scal(ins[3 + 3 * i])) for i in range(len(xs))],
                                 [int(scal(ins[4 + 3 * i])) for i in range(len(xs))],
                                 float(scal(ins[0])), int(scal(ins[1])))
            shp = list(xs[0].shape)
            if nhwc:
                shp[3] = sum(counts)
            else:
                shp[ax] = sum(x.shape[ax] for x in xs)
            y = y.reshape(shp)
        elif op == "MaxPool":
            src = graph.node_by_name(nd["name"])
            a = src.attrs
            x = val(ins[0])
            # (inside a fused chain the input is the producer's NHWC result,
            # under the graph's pre-fusion tensor name)
            assert (ins[0] in chain_env or fmt_of(ins[0]) == 1) and x.dtype == np.uint8
            k, s, p = a["kernel_shape"], a.get("strides", [1, 1]), a.get("pads", [0, 0, 0, 0])
            oH = (x.shape[1] + p[0] + p[2] - k[0]) // s[0] + 1
            oW = (x.shape[2] + p[1] + p[3] - k[1]) // s[1] + 1
            y = O.maxpool_u8_nhwc(x, k[0], k[1], s[0], s[1], p[0], p[1], oH, oW)
        elif op == "GlobalAveragePool":
            x = val(ins[0])
            if fmt_of(ins[0]):
                y = x.mean(axis=(1, 2), dtype=np.float64).astype(np.float32)[:, :, None, None]
            else:
                y = x.mean(axis=(2, 3), dtype=np.float64).astype(np.float32)[:, :, None, None]
            y = _nchw_to_phys(y, fmt_of(outs[0]))
        elif op in ("Flatten",):
            x = val(ins[0])
            ax = graph.node_by_name(nd["name"]).attrs.get("axis", 1)
            y = x.reshape(int(np.prod(x.shape[:ax])), -1)
        elif op == "Reshape":
            x = val(ins[0])
            shp = [int(v) for v in init[ins[1]]]
            shp = [x.shape[i] if v == 0 else v for i, v in enumerate(shp)]
            y = x.reshape(shp)
        elif op == "Gemm":
            a = graph.node_by_name(nd["name"]).attrs
            A = val(ins[0]).astype(np.float64)
            B = val(ins[1]).astype(np.float64)
            if a.get("transA", 0):
                A = A.T
            if a.get("transB", 0):
                B = B.T
            y = a.get("alpha", 1.0) * (A @ B)
            if len(ins) > 2 and ins[2]:
                y = y + a.get("beta", 1.0) * val(ins[2]).astype(np.float64)
            y = y.astype(np.float32)
        elif op == "ConvInteger":
            a = graph.node_by_name(nd["name"]).attrs
            x, w = val(ins[0]), val(ins[1])
            k = a.get("kernel_shape", list(w.shape[2:]))
            st, dl = a.get("strides", [1, 1]), a.get("dilations", [1, 1])
            pads = list(a.get("pads", [0, 0, 0, 0]))
            ap = a.get("auto_pad", "NOTSET")
            out = []
            for i in range(2):
                d, ke = x.shape[2 + i], (k[i] - 1) * dl[i] + 1
                if ap in ("SAME_UPPER", "SAME_LOWER"):
                    pad = (int(np.ceil(np.float32(d) / np.float32(st[i]))) - 1) * st[i] + ke - d
                    pads[i] = pad // 2 if ap == "SAME_UPPER" else pad - pad // 2
                    out.append(int(np.ceil(np.float32(d) / np.float32(st[i]))))
                elif ap == "VALID":
                    pads[i] = 0
                    out.append(int(np.ceil(np.float32(d - ke + 1) / np.float32(st[i]))))
                else:
                    out.append(int(np.floor(np.float32(d + pads[i] + pads[i + 2] - ke) / np.float32(st[i]) + 1)))
            wz = val(ins[3]).reshape(-1).astype(np.int32) if len(ins) > 3 and ins[3] else 0
            y = O.conv_integer(x, w, int(scal(ins[2])) if len(ins) > 2 and ins[2] else 0, wz, st, pads[:2], dl,
                               a.get("group", 1), out_hw=tuple(out))
        elif op == "BatchNormalization":
            # inference, fp32 (BatchNormalization.cpp:126-160), in float64
            x = val(ins[0]).astype(np.float64)
            sc, bias, mean, var = (val(t).astype(np.float64) for t in ins[1:5])
            eps = float(graph.node_by_name(nd["name"]).attrs.get("epsilon", 1e-5))
            shp = [1] * x.ndim
            shp[x.ndim - 1 if fmt_of(ins[0]) else 1] = -1
            r = lambda v: v.reshape(shp)
            y = ((x - r(mean)) / np.sqrt(r(var) + eps) * r(sc) + r(bias)).astype(np.float32)
        else:
            raise NotImplementedError(op)
        return {outs[0]: y, **extra}

    def folded_bn(nd):
        """fold_bn_qdq's BatchNormalization: A / B restated from the original
        BN, DQ and Q definitions (fold_bn_qdq.cpp:138-147, 230-236), then the
        folded kernel's per-layout rounding."""
        bn = graph.node_by_name(nd["name"])
        sc, bias, mean, var = (init[t] for t in bn.inputs[1:5])
        q = graph.node_by_name(nd["fused_chain"][-1])
        q_s = float(init[q.inputs[1]].reshape(-1)[0])
        q_zp = int(init[q.inputs[2]].reshape(-1)[0]) if len(q.inputs) > 2 and q.inputs[2] else 0
        dq = None
        if nd.get("fused_pre"):
            d = graph.node_by_name(nd["fused_pre"][0])
            dq = (float(init[d.inputs[1]].reshape(-1)[0]),
                  int(init[d.inputs[2]].reshape(-1)[0]) if len(d.inputs) > 2 and d.inputs[2] else 0)
        A, B = O.fold_bn(sc, bias, mean, var, float(bn.attrs.get("epsilon", 1e-5)), q_s, q_zp, dq=dq)
        x = val(nd["inputs"][0])
        return {nd["outputs"][0]: O.batchnorm_u8(x, A, B, nhwc=fmt_of(nd["inputs"][0]))}

    for nd in plan:
        if nd["op"] in skip_ops:
            continue
        if nd["op"] == "BatchNormalization" and nd.get("variant") in ("DQ-BN-Q", "BN-Q"):
            env.update(folded_bn(nd))
            if stop_after and nd["name"] == stop_after:
                break
            continue
        pre = nd.get("fused_pre") or []
        if pre:
            # nodes folded into this kernel before it: replay them from the
            # graph's definitions; this node then reads the last one's output
            # (its input 0 before the fusion)
            for name in pre:
                gn = graph.node_by_name(name)
                chain_env.update(exec_node({"op": gn.op, "name": gn.name, "inputs": list(gn.inputs),
                                            "outputs": list(gn.outputs), "post_fn": 0}))
            nd2 = dict(nd, inputs=[graph.node_by_name(pre[-1]).outputs[0]] + list(nd["inputs"][1:]))
            res = exec_node(nd2)
            if "oracle_branch" in nd2:
                nd["oracle_branch"] = nd2["oracle_branch"]
        else:
            res = exec_node(nd)
        chain = nd.get("fused_chain") or []
        if chain:
            # nodes folded into this kernel: the result above is the first
            # one's input; replay them in order from the graph's definitions
            first = graph.node_by_name(chain[0])
            chain_env[first.inputs[0]] = res[nd["outputs"][0]]
            # an fp32 producer's fused unary (fuse_post_ops) runs in its
            # post-op form, on the producer's own output buffer
            post_op = bool(nd.get("post_fn")) and nd["op"] in ("Gemm", "MatMul", "Conv")
            for name in chain:
                gn = graph.node_by_name(name)
                cres = exec_node({"op": gn.op, "name": gn.name, "inputs": list(gn.inputs),
                                  "outputs": list(gn.outputs), "post_fn": 0, "post_op": post_op})
                chain_env.update(cres)
            last = graph.node_by_name(chain[-1]).outputs[0]
            if last == nd["outputs"][0]:
                # the chain's last output is this node's own (a device tensor):
                # later nodes read it through `source` like any other output
                res = {nd["outputs"][0]: chain_env.pop(nd["outputs"][0])}
            else:
                # a fused post-op: its output is an alias of this node's
                v = chain_env.pop(last)
                res = {nd["outputs"][0]: v, last: v}
        env.update(res)
        if stop_after and nd["name"] == stop_after:
            break
    if keep_chain:
        env.update(chain_env)
    return env
