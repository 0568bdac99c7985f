"""The reference's CPU forward restated for the benchmark's CPU baseline (test infrastructure, as is all of oracle/).

Runs a parsed .knx model (knx_ref.parse) on the host with the oracle's plain-C kernels only, on its pthread pool of
`threads` workers (the reference's pool: 7 workers + the caller, reference include/kernix.h:63, src/kernix_runtime.c):
LINEAR as the fp32 native GEMM with its bias (reference include/kernix.h:108-124 via include/kernix_model.h:544-550),
int8 LINEAR weights as the reference dispatches them (the int8 kernel at <= 2 rows, include/kernix_model.h:99-182;
the dequantized fp32 copy above, :1616-1622), activations as a pass over the rows (:468-541), convolution as im2col
tiles and the native GEMM (:677-771), layer_norm and softmax row by row (include/kernix.h:652-677), attention as the
three projections, the per-(batch, head) scores / softmax / context loop and the output projection (:1005-1048),
broadcasting binaries and global pooling (:810-906), recurrent layers as the input-projection GEMM and the
per-timestep h·U and gates (:563-648).  Only the op kinds of the benchmark models are covered;
anything else raises.  Accuracy is the reference's, not the oracle's float64: this is a baseline to time, not a
checker.
"""
import numpy as np

from . import knx_ref

INT8_MAX_ROWS = 2


def _p(a):
    return knx_ref._p(a)


def _dense(x, w, b, act_id=-1):
    L = knx_ref.lib()
    M, K = x.shape
    N = w.shape[1]
    y = np.empty((M, N), np.float32)
    L.ko_dense(M, N, K, _p(x), _p(np.ascontiguousarray(w, np.float32)), _p(None if b is None else knx_ref.f32c(b)),
               act_id, 0.0, _p(y))
    return y


def _act(y, act_id, alpha):
    knx_ref.lib().ko_act(_p(y), y.size, act_id, float(alpha))
    return y


class CpuModel:
    """A model prepared once (fp32 copies of int8 weights, as the reference's workspace keeps them) and run on x."""

    def __init__(self, model):
        self.m = model
        self.deq = {}
        for i, op in enumerate(model["ops"]):
            if op["kind"] == 0 and op["w"][0] == "i8":
                q, sc = op["w"][1], op["w"][2]
                self.deq[i] = np.ascontiguousarray(q.astype(np.float32) * sc[None, :])

    def forward(self, x, threads):
        L = knx_ref.lib()
        old = L.ko_get_threads()
        L.ko_set_threads(int(threads))
        try:
            return self._run(np.ascontiguousarray(x, np.float32))
        finally:
            L.ko_set_threads(old)

    def _run(self, x):
        L = knx_ref.lib()
        in_shape = self.m["in_shape"]
        B = x.shape[0] // knx_ref._shape_rows(in_shape)
        vals, shapes = [x], [tuple(in_shape)]
        for i, op in enumerate(self.m["ops"]):
            k = op["kind"]
            a, sa = vals[op["inp"][0]], shapes[op["inp"][0]]
            if k == 0:  # LINEAR
                w = op["w"]
                if w[0] == "i8" and a.shape[0] <= INT8_MAX_ROWS:
                    y = knx_ref.qmatmul(a, w[1], w[2], op["b"])
                else:
                    y = _dense(a, self.deq[i] if w[0] == "i8" else w[1], op["b"])
                s = sa[:-1] + (op["n"],)
            elif k == 1:  # ACT
                y, s = _act(a.copy(), op["act"], op["alpha"]), sa
            elif k == 2:
                y, s = knx_ref.layernorm(a, op["g"], op["b"], op["eps"]), sa
            elif k == 3:
                y, s = knx_ref.softmax(a), sa
            elif k == 7:  # CONV
                H, W = sa[0], (sa[1] if len(sa) == 3 else 1)
                kh, kw = op["k"]
                (sh, sw), (dh, dw), (pt, pb, pl, pr) = op["s"], op["d"], op["p"]
                Ho = (H + pt + pb - dh * (kh - 1) - 1) // sh + 1
                Wo = (W + pl + pr - dw * (kw - 1) - 1) // sw + 1
                y = np.empty((B * Ho * Wo, op["cout"]), np.float32)
                L.ko_conv(B, H, W, op["cin"], Ho, Wo, op["cout"], kh, kw, sh, sw, dh, dw, pt, pl, op["g"], _p(a),
                          _p(knx_ref.f32c(op["w"])), _p(None if op["b"] is None else knx_ref.f32c(op["b"])), -1, 0.0,
                          _p(y))
                s = (Ho, Wo, op["cout"]) if len(sa) == 3 else (Ho, op["cout"])
            elif k == 9:  # GLOBAL_POOL
                R, C = knx_ref._shape_rows(sa), sa[-1]
                y = np.empty((B, C), np.float32)
                L.ko_global_pool(op["type"], _p(a), B, R, C, _p(y))
                s = (C,)
            elif k == 12:  # BINARY
                b, sb = vals[op["inp"][1]], shapes[op["inp"][1]]
                ra, rb = knx_ref._shape_rows(sa), knx_ref._shape_rows(sb)
                R, C = max(ra, rb), max(sa[-1], sb[-1])
                y = np.empty((B * R, C), np.float32)
                L.ko_binary(op["op"], _p(a), ra, sa[-1], _p(b), rb, sb[-1], _p(y), B, R, C)
                s = (sa if ra * sa[-1] >= rb * sb[-1] else sb)[:-1] + (C,)
            elif k in (4, 5, 6):  # LSTM / GRU / RNN: the input projection and the fp32 recurrence on the native
                # GEMM, int8 recurrences at <= 2 rows on the int8 kernel, the gates in float32 (include/kernix_model.h:563-648)
                y, s = knx_ref._rnn(op, a, sa, B, "ref", dense=lambda x, w, b: _dense(x, w, b))
            elif k == 17:  # ATTENTION
                y, s = self._attention(op, vals, shapes, B)
            else:
                raise ValueError(f"op kind {k} is not part of the benchmark models")
            vals.append(y)
            shapes.append(tuple(s))
        return vals[-1].reshape(B, -1)

    @staticmethod
    def _attention(op, vals, shapes, B):
        inp = op["inp"]
        vi = inp[1] if len(inp) > 1 else inp[0]
        ki = inp[2] if len(inp) > 2 else vi
        Rq, S = knx_ref._shape_rows(shapes[inp[0]]), knx_ref._shape_rows(shapes[vi])
        H, dk, dv = op["H"], op["dk"], op["dv"]
        (wq, bq), (wk, bk), (wv, bv), (wo, bo) = op["ws"]
        Q = _dense(vals[inp[0]], wq, bq)
        K = _dense(vals[ki], wk, bk)
        V = _dense(vals[vi], wv, bv)
        ctx = np.empty((B * Rq, H * dv), np.float32)
        knx_ref.lib().ko_attention_core(_p(Q), _p(K), _p(V), _p(ctx), B, H, Rq, S, dk, dv,
                                        float(np.float32(1.0) / np.sqrt(np.float32(dk))), int(op["causal"]))
        return _dense(ctx, wo, bo), shapes[inp[0]][:-1] + (wo.shape[1],)
