"""Graph construction and execution through the host framework's C ABI
(include/nnr_host.h, nnr_amd/lib/libnnr_host.so).

`Graph` collects initializers / inputs / outputs / nodes (what an ONNX
loader would produce); `Session` hands them to a C++ context_t with the HIP
backend preferred, prepares it (QDQ fusion, layout assignment, device
memory) and runs it on a stream.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

from . import _lib

_HERE = os.path.dirname(os.path.abspath(__file__))
HOST_LIB = os.path.join(_HERE, "lib", "libnnr_host.so")

ONNX_DT = {np.dtype(np.float32): 1, np.dtype(np.uint8): 2, np.dtype(np.int8): 3,
           np.dtype(np.int32): 6, np.dtype(np.int64): 7, np.dtype(np.float16): 10}
# the reference's data_type_t codes (src/nnr.h:20-56), which the host C ABI takes
NNR_DT = {np.dtype(np.float32): 1, np.dtype(np.float16): 3, np.dtype(np.int8): 5,
          np.dtype(np.int32): 7, np.dtype(np.int64): 8, np.dtype(np.uint8): 9}
NP_DT = {v: k for k, v in NNR_DT.items()}
BACKEND_HIP = 4

_hl = None


def host_lib():
    global _hl
    if _hl is None:
        _lib.lib()          # the HIP library must be loadable first
        if not os.path.exists(HOST_LIB):
            raise ImportError(f"{HOST_LIB} is missing: run __graft_entry__.build() first")
        L = C.CDLL(HOST_LIB)
        vp, i, cp = C.c_void_p, C.c_int, C.c_char_p
        P = C.POINTER
        sig = {
            "nnr_last_error": (cp, []),
            "nnr_ctx_create": (i, [P(vp), i]),
            "nnr_ctx_destroy": (i, [vp]),
            "nnr_ctx_set_stream": (i, [vp, vp]),
            "nnr_ctx_set_fusion": (i, [vp, i]),
            "nnr_ctx_set_graph": (i, [vp, i]),
            "nnr_ctx_graph_active": (i, [vp, P(i)]),
            "nnr_ctx_set_conv_add": (i, [vp, i]),
            "nnr_ctx_set_codes": (i, [vp, i]),
            "nnr_ctx_add_initializer": (i, [vp, cp, i, P(i), i, vp]),
            "nnr_ctx_add_input": (i, [vp, cp, i, P(i), i]),
            "nnr_ctx_add_output": (i, [vp, cp]),
            "nnr_ctx_add_node": (i, [vp, cp, cp, i, P(cp), i, P(cp), i, P(cp), P(i), P(i), P(i),
                                     P(C.c_int64), P(C.c_float), P(cp)]),
            "nnr_ctx_optimize": (i, [vp]),
            "nnr_ctx_prepare": (i, [vp]),
            "nnr_ctx_run": (i, [vp]),
            "nnr_group_create": (i, [P(vp), i, P(vp)]),
            "nnr_group_run": (i, [vp, vp]),
            "nnr_group_destroy": (i, [vp]),
            "nnr_ctx_tensor": (i, [vp, cp, P(vp), P(i), P(i), P(i), P(i)]),
            "nnr_ctx_node_count": (i, [vp, P(i)]),
            "nnr_ctx_node_info": (i, [vp, i, P(cp), P(cp), P(cp), P(i), P(i), P(i)]),
            "nnr_ctx_node_io": (i, [vp, i, i, i, P(cp)]),
            "nnr_ctx_node_fused_add": (i, [vp, i, i, P(cp)]),
            "nnr_ctx_node_fused_chain": (i, [vp, i, i, P(cp)]),
            "nnr_ctx_node_fused_pre": (i, [vp, i, i, P(cp)]),
            "nnr_ctx_fusion_stat": (i, [vp, cp, P(i)]),
            "nnr_ctx_device_bytes": (C.c_size_t, [vp]),
            "nnr_ctx_workspace_bytes": (C.c_size_t, [vp]),
            "nnr_ctx_set_memory_planning": (i, [vp, i]),
            "nnr_ctx_load_onnx": (i, [vp, vp, C.c_size_t, cp, i]),
            "nnr_ctx_load_onnx_file": (i, [vp, cp, i]),
            "nnr_ctx_graph_io_count": (i, [vp, i, P(i)]),
            "nnr_ctx_initializer": (i, [vp, cp, P(vp), P(C.c_size_t)]),
            "nnr_ctx_graph_io": (i, [vp, i, i, P(cp)]),
            "nnr_ctx_plan_memory": (i, [vp]),
            "nnr_ctx_memory_stats": (i, [vp, P(i), P(i), P(i), P(i), P(C.c_ulonglong), P(C.c_ulonglong)]),
            "nnr_ctx_memory_entry": (i, [vp, i, P(cp), P(i), P(i), P(C.c_ulonglong), P(C.c_ulonglong),
                                         P(i), P(i)]),
            "nnr_ctx_enable_profiling": (i, [vp, i]),
            "nnr_ctx_profile": (i, [vp, i, P(C.c_double), P(i), P(C.c_double), P(C.c_double)]),
            "nnr_ctx_time_node": (i, [vp, i, i, P(C.c_double)]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _hl = L
    return _hl


class NnrError(RuntimeError):
    pass


def _chk(rc):
    if rc != 0:
        raise NnrError(host_lib().nnr_last_error().decode())


@dataclass
class Node:
    op: str
    name: str
    inputs: list
    outputs: list
    attrs: dict = field(default_factory=dict)


class Graph:
    def __init__(self):
        self.initializers: dict[str, np.ndarray] = {}
        self.inputs: dict[str, tuple] = {}      # name -> (dtype, shape)
        self.outputs: list[str] = []
        self.nodes: list[Node] = []
        self._n = 0

    def init(self, name, arr):
        self.initializers[name] = np.ascontiguousarray(arr)
        return name

    def node(self, op, inputs, outputs=None, name=None, **attrs):
        self._n += 1
        name = name or f"{op}_{self._n}"
        if outputs is None:
            outputs = [f"{name}_out"]
        elif isinstance(outputs, str):
            outputs = [outputs]
        self.nodes.append(Node(op, name, list(inputs), list(outputs), attrs))
        return outputs[0] if len(outputs) == 1 else outputs

    def node_by_name(self, name):
        for n in self.nodes:
            if n.name == name:
                return n
        return None


def _attr_arrays(attrs: dict):
    names, kinds, counts, offs, ints, floats, strs = [], [], [], [], [], [], []
    for k, v in attrs.items():
        names.append(k.encode())
        if isinstance(v, str):
            kinds.append(2); counts.append(0); offs.append(0); strs.append(v.encode())
            continue
        strs.append(None)
        if isinstance(v, (list, tuple, np.ndarray)):
            vals = list(v)
            if all(isinstance(x, (int, np.integer)) for x in vals):
                kinds.append(3); counts.append(len(vals)); offs.append(len(ints))
                ints.extend(int(x) for x in vals)
            else:
                kinds.append(4); counts.append(len(vals)); offs.append(len(floats))
                floats.extend(float(x) for x in vals)
        elif isinstance(v, (int, np.integer)):
            kinds.append(0); counts.append(1); offs.append(len(ints)); ints.append(int(v))
        else:
            kinds.append(1); counts.append(1); offs.append(len(floats)); floats.append(float(v))
    n = len(names)
    A = lambda T, xs: (T * max(1, len(xs)))(*xs)
    return (n, A(C.c_char_p, names), A(C.c_int, kinds), A(C.c_int, counts), A(C.c_int, offs),
            A(C.c_int64, ints), A(C.c_float, floats), A(C.c_char_p, strs))


class Session:
    """A prepared C++ context_t for `graph` with the HIP backend preferred."""

    def __init__(self, graph: Graph | None, stream=None, fusion=True, device=True, conv_add=True,
                 memory_planning=False, onnx=None, sym_dim=0, hip_graph=True, codes=True):
        """graph: the in-process description, built into the context through
        the C ABI. onnx: instead, an ONNX model -- a file path (external data
        relative to it) or ModelProto bytes -- loaded by the C++ loader;
        sym_dim: the value of symbolic input dimensions (0: 1). hip_graph:
        from the second run() on, replay the plan as one captured HIP graph.
        codes: a fused dequantize chain read only by an operator that can
        form its values from the uint8 QLinearMatMul bytes (DynamicQuantizeLinear,
        LayerNormalization, MultiHeadAttention) stores those bytes (that
        tensor reads back as uint8) instead of its fp32 values."""
        L = host_lib()
        self.L = L
        self.graph = graph
        h = C.c_void_p()
        _chk(L.nnr_ctx_create(C.byref(h), BACKEND_HIP))
        self.h = h
        if stream is None and device:
            stream = _lib.cur_stream()
        self.stream = stream
        _chk(L.nnr_ctx_set_stream(h, stream))
        _chk(L.nnr_ctx_set_fusion(h, 1 if fusion else 0))
        _chk(L.nnr_ctx_set_graph(h, 1 if hip_graph else 0))
        _chk(L.nnr_ctx_set_conv_add(h, 1 if conv_add else 0))
        _chk(L.nnr_ctx_set_codes(h, 1 if codes else 0))
        _chk(L.nnr_ctx_set_memory_planning(h, 1 if memory_planning else 0))
        if onnx is not None:
            if isinstance(onnx, (bytes, bytearray)):
                buf = C.create_string_buffer(bytes(onnx), len(onnx))
                _chk(L.nnr_ctx_load_onnx(h, buf, len(onnx), None, sym_dim))
            else:
                _chk(L.nnr_ctx_load_onnx_file(h, os.fsencode(onnx), sym_dim))
            _chk(L.nnr_ctx_prepare(h) if device else L.nnr_ctx_optimize(h))
            return
        for name, arr in graph.initializers.items():
            dims = (C.c_int * max(1, arr.ndim))(*arr.shape)
            _chk(L.nnr_ctx_add_initializer(h, name.encode(), NNR_DT[arr.dtype], dims, arr.ndim,
                                           arr.ctypes.data))
        for name, (dt, shape) in graph.inputs.items():
            dims = (C.c_int * max(1, len(shape)))(*shape)
            _chk(L.nnr_ctx_add_input(h, name.encode(), NNR_DT[np.dtype(dt)], dims, len(shape)))
        for name in graph.outputs:
            _chk(L.nnr_ctx_add_output(h, name.encode()))
        for nd in graph.nodes:
            ins = (C.c_char_p * max(1, len(nd.inputs)))(*[s.encode() if s else None for s in nd.inputs])
            outs = (C.c_char_p * max(1, len(nd.outputs)))(*[s.encode() for s in nd.outputs])
            na, an, ak, ac, ao, ai, af, as_ = _attr_arrays(nd.attrs)
            _chk(L.nnr_ctx_add_node(h, nd.op.encode(), nd.name.encode(), len(nd.inputs), ins,
                                    len(nd.outputs), outs, na, an, ak, ac, ao, ai, af, as_))
        # device=False: graph passes + shapes + layouts only (no GPU needed)
        _chk(L.nnr_ctx_prepare(h) if device else L.nnr_ctx_optimize(h))

    # ---- data ---------------------------------------------------------------
    def tensor_info(self, name):
        p, dt, nd, fmt = C.c_void_p(), C.c_int(), C.c_int(), C.c_int()
        dims = (C.c_int * 8)()
        _chk(self.L.nnr_ctx_tensor(self.h, name.encode(), C.byref(p), C.byref(dt), dims,
                                   C.byref(nd), C.byref(fmt)))
        return p.value, NP_DT.get(dt.value), tuple(dims[:nd.value]), fmt.value

    def set_input(self, name, arr):
        """Copy a host numpy array or a device torch tensor into a graph tensor."""
        p, dt, shape, fmt = self.tensor_info(name)
        if isinstance(arr, np.ndarray):
            a = np.ascontiguousarray(arr, dtype=dt)
            assert a.size == int(np.prod(shape)), (a.shape, shape)
            _lib.check(_lib.lib().nnrh_memcpy(p, a.ctypes.data, a.nbytes, 0, _lib.cur_stream()))
            _lib.check(_lib.lib().nnrh_stream_synchronize(_lib.cur_stream()))
        else:
            nbytes = arr.numel() * arr.element_size()
            assert arr.is_contiguous() and arr.numel() == int(np.prod(shape))
            _lib.check(_lib.lib().nnrh_memcpy(p, arr.data_ptr(), nbytes, 2, _lib.cur_stream()))
            if self.stream != _lib.cur_stream():
                # the context runs on a stream of its own: the copy lands first
                _lib.check(_lib.lib().nnrh_stream_synchronize(_lib.cur_stream()))

    def output(self, name):
        """numpy copy of a tensor in its physical layout, plus the layout flag
        (1 = NHWC: a 4-D tensor comes back as [N, H, W, C])."""
        p, dt, shape, fmt = self.tensor_info(name)
        phys = shape
        if fmt == 1 and len(shape) == 4:
            phys = (shape[0], shape[2], shape[3], shape[1])
        out = np.empty(phys, dtype=dt)
        _lib.check(_lib.lib().nnrh_stream_synchronize(_lib.cur_stream()))
        if self.stream and self.stream != _lib.cur_stream():
            _lib.check(_lib.lib().nnrh_stream_synchronize(self.stream))
        _lib.check(_lib.lib().nnrh_memcpy(out.ctypes.data, p, out.nbytes, 1, _lib.cur_stream()))
        return out, fmt

    def run(self):
        _chk(self.L.nnr_ctx_run(self.h))

    # ---- plan introspection ------------------------------------------------------
    def plan(self):
        L = self.L
        n = C.c_int()
        _chk(L.nnr_ctx_node_count(self.h, C.byref(n)))
        out = []
        for i in range(n.value):
            op, nm, var = C.c_char_p(), C.c_char_p(), C.c_char_p()
            pf, ni, no = C.c_int(), C.c_int(), C.c_int()
            _chk(L.nnr_ctx_node_info(self.h, i, C.byref(op), C.byref(nm), C.byref(var),
                                     C.byref(pf), C.byref(ni), C.byref(no)))
            ios = []
            for is_out, cnt in ((0, ni.value), (1, no.value)):
                lst = []
                for j in range(cnt):
                    s = C.c_char_p()
                    _chk(L.nnr_ctx_node_io(self.h, i, is_out, j, C.byref(s)))
                    lst.append(s.value.decode())
                ios.append(lst)
            def fused(j):
                s = C.c_char_p()
                _chk(L.nnr_ctx_node_fused_add(self.h, i, j, C.byref(s)))
                return s.value.decode()
            fadd = None
            if fused(-1):
                fadd = dict(name=fused(-1), other=fused(-2), inputs=[fused(j) for j in range(8)])
            chain = []
            while True:
                c = C.c_char_p()
                _chk(L.nnr_ctx_node_fused_chain(self.h, i, len(chain), C.byref(c)))
                if not c.value:
                    break
                chain.append(c.value.decode())
            pre = []
            while True:
                c = C.c_char_p()
                _chk(L.nnr_ctx_node_fused_pre(self.h, i, len(pre), C.byref(c)))
                if not c.value:
                    break
                pre.append(c.value.decode())
            out.append(dict(op=op.value.decode(), name=nm.value.decode(), variant=var.value.decode(),
                            post_fn=pf.value, inputs=ios[0], outputs=ios[1], fused_add=fadd,
                            fused_chain=chain, fused_pre=pre))
        return out

    def fusion_stat(self, key):
        v = C.c_int()
        _chk(self.L.nnr_ctx_fusion_stat(self.h, key.encode(), C.byref(v)))
        return v.value

    def initializer_bytes(self, name):
        """The context's host copy of an initializer, as bytes."""
        p, n = C.c_void_p(), C.c_size_t()
        _chk(self.L.nnr_ctx_initializer(self.h, name.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p.value, n.value) if p.value else b""

    def graph_io(self, outputs=True):
        """Names of the context's graph outputs (or inputs), in order."""
        n = C.c_int()
        _chk(self.L.nnr_ctx_graph_io_count(self.h, 1 if outputs else 0, C.byref(n)))
        out = []
        for k in range(n.value):
            nm = C.c_char_p()
            _chk(self.L.nnr_ctx_graph_io(self.h, 1 if outputs else 0, k, C.byref(nm)))
            out.append(nm.value.decode())
        return out

    def device_bytes(self):
        return int(self.L.nnr_ctx_device_bytes(self.h))

    def workspace_bytes(self):
        """Bytes of the operators' shared scratch buffer (0: none needed)."""
        return int(self.L.nnr_ctx_workspace_bytes(self.h))

    def memory_plan(self):
        """The memory plan: (stats dict, entries). Without a prepared device
        context this plans the optimized graph without allocating. Entry:
        dict(name, first, last, offset, bytes, kind 'slot'|'inplace'|'concat',
        parent index or -1); first / last are node positions."""
        L = self.L
        _chk(L.nnr_ctx_plan_memory(self.h))
        a, b, c, d = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        pb, ub = C.c_ulonglong(), C.c_ulonglong()
        _chk(L.nnr_ctx_memory_stats(self.h, C.byref(a), C.byref(b), C.byref(c), C.byref(d),
                                    C.byref(pb), C.byref(ub)))
        stats = dict(intermediates=a.value, slots=b.value, inplace=c.value, concat=d.value,
                     pool_bytes=pb.value, unpooled_bytes=ub.value)
        entries = []
        kinds = ("slot", "inplace", "concat")
        for k in range(a.value):
            nm, f, l_, o, by, kd, par = (C.c_char_p(), C.c_int(), C.c_int(), C.c_ulonglong(),
                                         C.c_ulonglong(), C.c_int(), C.c_int())
            _chk(L.nnr_ctx_memory_entry(self.h, k, C.byref(nm), C.byref(f), C.byref(l_), C.byref(o),
                                        C.byref(by), C.byref(kd), C.byref(par)))
            entries.append(dict(name=nm.value.decode(), first=f.value, last=l_.value, offset=o.value,
                                bytes=by.value, kind=kinds[kd.value], parent=par.value))
        return stats, entries

    def graph_active(self) -> bool:
        """True once run() replays a captured HIP graph."""
        on = C.c_int()
        _chk(self.L.nnr_ctx_graph_active(self.h, C.byref(on)))
        return bool(on.value)

    def enable_profiling(self, on=True):
        _chk(self.L.nnr_ctx_enable_profiling(self.h, 1 if on else 0))

    def profile(self):
        rows = []
        for i, p in enumerate(self.plan()):
            ms, runs, ops, nb = C.c_double(), C.c_int(), C.c_double(), C.c_double()
            _chk(self.L.nnr_ctx_profile(self.h, i, C.byref(ms), C.byref(runs), C.byref(ops),
                                        C.byref(nb)))
            rows.append(dict(p, ms=ms.value, runs=runs.value, ops=ops.value, bytes=nb.value))
        return rows

    def time_node(self, i, reps=10):
        """Average ms of plan node i run `reps` times back to back."""
        ms = C.c_double()
        _chk(self.L.nnr_ctx_time_node(self.h, i, reps, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if getattr(self, "h", None):
                self.L.nnr_ctx_destroy(self.h)
                self.h = None
        except Exception:
            pass


class SplitSession:
    """A batch split into `parts` slices along axis 0, one prepared context
    per slice (built for batch / parts), run concurrently as one step
    (nnr_group_run): each context on a stream of its own, so one slice's
    short, latency-bound launches fill the CUs the other slices leave idle.
    Every slice's results are those of running it alone, and the plan is the
    same for every slice. make_graph(batch) builds a slice's graph; or onnx=
    (a file or bytes), loaded with the slice's batch as the symbolic
    dimension. set_input / output take and give the whole batch; run()
    enqueues one step on the current stream: the slices start after the work
    already on it, and its later work waits for all of them."""

    def __init__(self, make_graph=None, batch=0, parts=2, onnx=None, **kw):
        if parts < 1 or batch < parts or batch % parts:
            raise ValueError(f"batch {batch} does not split into {parts} equal parts")
        self.parts, self.batch, self.sub = parts, batch, batch // parts
        self.streams, self.sessions, self.g = [], [], None
        L = _lib.lib()
        for _ in range(parts):
            st = C.c_void_p()
            _lib.check(L.nnrh_stream_create(C.byref(st)))
            self.streams.append(st.value)
            if onnx is not None:
                self.sessions.append(Session(None, stream=st.value, onnx=onnx, sym_dim=self.sub, **kw))
            else:
                self.sessions.append(Session(make_graph(self.sub), stream=st.value, **kw))
        hs = (C.c_void_p * parts)(*[s.h.value for s in self.sessions])
        g = C.c_void_p()
        _chk(host_lib().nnr_group_create(hs, parts, C.byref(g)))
        self.g = g

    def slice(self, k):
        return slice(k * self.sub, (k + 1) * self.sub)

    def set_input(self, name, arr):
        for k, s in enumerate(self.sessions):
            s.set_input(name, arr[self.slice(k)])

    def output(self, name):
        outs = [s.output(name) for s in self.sessions]
        return np.concatenate([o for o, _ in outs], axis=0), outs[0][1]

    def run(self):
        _chk(host_lib().nnr_group_run(self.g, _lib.cur_stream()))

    def plan(self):
        return self.sessions[0].plan()

    def graph_active(self) -> bool:
        return all(s.graph_active() for s in self.sessions)

    def device_bytes(self):
        return sum(s.device_bytes() for s in self.sessions)

    def close(self):
        L = _lib.lib()
        for st in self.streams:
            L.nnrh_stream_synchronize(st)
        if self.g:
            host_lib().nnr_group_destroy(self.g)
            self.g = None
        self.sessions = []          # the contexts go before their streams
        import gc
        gc.collect()
        for st in self.streams:
            L.nnrh_stream_destroy(st)
        self.streams = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

