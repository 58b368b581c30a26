"""Config-3 decode step of the quantized linear path, driven through the C ABI.

A stack of `layers` weight sets applied `passes` times (the reference's
looped 22-layer model: 44 slots, each weight set read twice), then the final
norm, the bf16 LM head and the greedy token.  Per slot, the linear-path
launches of the reference engine's decode step
(include/viper/model_impl.cuh:650-728), attention itself excluded (it is not
on this path; its output is a fixed activation):

    rmsnorm_quantize(x, input_ln)  -> q GEMV, fused2(k, v)
    quantize(attn)                 -> o GEMV + residual (in place on x)
    rmsnorm_quantize(x, post_ln)   -> fused2(gate, up)
    swiglu_quantize(gate, up)      -> down GEMV + residual (in place on x)

step_fused() is the same computation in 4 launches per slot instead of 9:
the producers are folded into the GEMV prologues, q/k/v are one launch over
their concatenated weight (each layer stores q, k and v row after row, the
engine's fused qkv matrix; viper_hip_qlinear_m1), and the gate/up launch pairs
the rows of both matrices
so its epilogue writes h = silu(gate) * up (viper_hip_qlinear_m1_swiglu,
bit-identical to the swiglu of the two outputs); the down projection then
quantizes h in its prologue:

    [rmsnorm(x, input_ln) -> q, k, v]          [quantize(attn) -> o + residual]
    [rmsnorm(x, post_ln) -> gate, up -> h]     [quantize(h) -> down + residual]

Device buffers are torch tensors (allocation only); every launch is a C ABI
call on the current stream, so a whole step can be captured in a HIP graph.
"""
import ctypes as C
import math

from . import qlinear as _q

Q4 = int(_q.QType.Q4_G64)


class Stack:
    def __init__(self, torch, hidden=2560, inter=10240, n_heads=20, n_kv_heads=4, head_dim=128,
                 layers=22, passes=2, vocab=166144, seed=0x5EED0003, eps=1e-6):
        self.torch = torch
        self.H, self.I = hidden, inter
        self.nQ, self.nKV = n_heads * head_dim, n_kv_heads * head_dim
        self.layers, self.passes, self.V, self.eps = layers, passes, vocab, eps
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.gen = g
        H, I, nQ, nKV = self.H, self.I, self.nQ, self.nKV
        shapes = [(nQ, H), (nKV, H), (nKV, H), (H, nQ), (I, H), (I, H), (H, I)]
        self.w = []        # per layer: 7 (packed, scales, N, K), views of the layer's arena
        self.wqkv = []     # per layer: q, k and v as one matrix of nQ + 2 nKV rows (views of the same bytes)
        self.arenas = []   # per layer: one device buffer, every section at a 256-byte aligned offset
        sec = lambda nbytes: (nbytes + 255) // 256 * 256
        # q, k and v lie row after row in one packed section and one scale section, so the fused
        # step reads them as one matrix (the engine's concatenated qkv weight): a launch with one
        # matrix keeps every workgroup's arguments among the preloaded ones
        nqkv = nQ + 2 * nKV
        assert (nQ * (H // 64) * 2) % 16 == 0 and (nKV * (H // 64) * 2) % 16 == 0, "16-byte aligned q/k/v scales"
        for _ in range(layers):
            sizes = [sec(nqkv * H // 2), sec(nqkv * (H // 64) * 2)] + \
                    [sec(n * k // 2) + sec(n * (k // 64) * 2) for n, k in shapes[3:]]
            arena = torch.empty(sum(sizes), dtype=torch.uint8, device="cuda")
            lw = []
            qkv_p, qkv_s = arena[:nqkv * H // 2], arena[sizes[0]:sizes[0] + nqkv * (H // 64) * 2].view(torch.float16)
            prow, srow = 0, 0
            for (n, k) in shapes[:3]:
                packed = qkv_p[prow * (k // 2):(prow + n) * (k // 2)]
                packed.copy_(torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device="cuda", generator=g))
                u = torch.rand((n * (k // 64),), device="cuda", generator=g)
                scales = qkv_s[srow * (k // 64):(srow + n) * (k // 64)]
                scales.copy_(torch.exp(math.log(1e-3) + u * math.log(10.0)).to(torch.float16))
                prow += n
                srow += n
                lw.append((packed, scales, n, k))
            off = sizes[0] + sizes[1]
            for (n, k) in shapes[3:]:
                packed = arena[off:off + n * k // 2]
                packed.copy_(torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device="cuda", generator=g))
                off += sec(n * k // 2)
                u = torch.rand((n * (k // 64),), device="cuda", generator=g)
                scales = arena[off:off + n * (k // 64) * 2].view(torch.float16)
                scales.copy_(torch.exp(math.log(1e-3) + u * math.log(10.0)).to(torch.float16))
                off += sec(n * (k // 64) * 2)
                lw.append((packed, scales, n, k))
            self.w.append(lw)
            self.wqkv.append((qkv_p, qkv_s, nqkv, H))
            self.arenas.append(arena)
        bf = torch.bfloat16
        self.ln = [(1.0 + 0.05 * torch.randn((H,), device="cuda", generator=g)).to(bf) for _ in range(2 * layers)]
        self.final_ln = (1.0 + 0.05 * torch.randn((H,), device="cuda", generator=g)).to(bf)
        self.head = (0.02 * torch.randn((vocab, H), device="cuda", generator=g)).to(bf)
        self.x0 = torch.randn((1, H), device="cuda", generator=g).to(bf)
        self.attn = torch.randn((1, nQ), device="cuda", generator=g).to(bf)
        self.x = torch.empty((1, H), dtype=bf, device="cuda")
        self.qkv = torch.empty((1, nQ + 2 * nKV), dtype=bf, device="cuda")
        self.q = self.qkv[:, :nQ]
        self.k = self.qkv[:, nQ:nQ + nKV]
        self.v = self.qkv[:, nQ + nKV:]
        self.gt = torch.empty((1, I), dtype=bf, device="cuda")
        self.ut = torch.empty((1, I), dtype=bf, device="cuda")
        self.xn = torch.empty((1, H), dtype=bf, device="cuda")
        kmax = max(H, I, nQ)
        self.xq = torch.empty((kmax,), dtype=torch.int8, device="cuda")
        self.xs = torch.empty((kmax // 64,), dtype=torch.float32, device="cuda")
        self.logits = torch.empty((1, vocab), dtype=bf, device="cuda")
        self.token = torch.empty((1,), dtype=torch.int32, device="cuda")
        # the split greedy pick's workspace: zero once, every call leaves it zero
        self.greedy_ws = torch.zeros((16,), dtype=torch.uint8, device="cuda")
        # trace: every launch also leaves its intermediates readable (the
        # normalized rows in xn, gate in g, up in ut, h in gt) through the same
        # kernels' optional outputs, so a test can check each launch in turn
        self.trace = False
        self.g = torch.empty((1, I), dtype=bf, device="cuda")
        # MALL warming of the next slot's weights from a second stream (default priority)
        self.side = None
        self.sink = torch.zeros((1,), dtype=torch.int32, device="cuda")
        L = _q.lib()
        self.L = L

    def weight_bytes_per_step(self):
        per_layer = sum(p.numel() + s.numel() * 2 for (p, s, _, _) in self.w[0])
        return per_layer * self.layers * self.passes + self.head.numel() * 2

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    def _norm_out(self, pro):
        return self.xn.data_ptr() if self.trace and pro == 2 else None

    def _m1(self, pro, a, b, outs, eps=0.0, residual=None, st=None):
        n = len(outs)
        vp = C.c_void_p * n
        rc = self.L.viper_hip_qlinear_m1(Q4, 0, 64, outs[0][0][3], pro, a, b, eps, self._norm_out(pro), n,
                                         vp(*[o[0][0].data_ptr() for o in outs]),
                                         vp(*[o[0][1].data_ptr() for o in outs]),
                                         (C.c_int * n)(*[o[0][2] for o in outs]),
                                         vp(*[o[1].data_ptr() for o in outs]), residual, st)
        self._ok(rc, "qlinear_m1")

    def _m1_swiglu(self, pro, a, b, wg, wu, h, eps=0.0, st=None):
        gu = (self.g.data_ptr(), self.ut.data_ptr()) if self.trace else (None, None)
        rc = self.L.viper_hip_qlinear_m1_swiglu(Q4, 0, 64, wg[3], pro, a, b, eps, self._norm_out(pro),
                                                wg[0].data_ptr(), wg[1].data_ptr(), wu[0].data_ptr(),
                                                wu[1].data_ptr(), wg[2], h.data_ptr(), gu[0], gu[1], st)
        self._ok(rc, "qlinear_m1_swiglu")

    def attention_half(self, l, fused=True):
        """Slot l's q/k/v projections from rmsnorm(x) and the o projection of
        the fixed attention output added into x.  Slot 0 reads the step's input
        row x0 (the embedding's output) and its o projection writes x, so a
        step needs no copy of x0 into x."""
        L, st = self.L, self.torch.cuda.current_stream().cuda_stream
        H, nQ, nKV = self.H, self.nQ, self.nKV
        p = lambda t: t.data_ptr()
        x = self.x
        xin = self.x0 if l == 0 else x
        wq, wk, wv, wo = self.w[l % self.layers][:4]
        ln = self.ln[2 * (l % self.layers)]
        if fused:
            self._m1(2, p(xin), p(ln), [(self.wqkv[l % self.layers], self.qkv)], eps=self.eps, st=st)
            self._m1(0, p(self.attn), None, [(wo, x)], residual=p(xin), st=st)
            return
        self._ok(L.viper_hip_rmsnorm_quantize(p(xin), p(ln), self.eps, 1, H, 64, p(self.xn), p(self.xq),
                                              p(self.xs), st), "rmsnorm_quantize")
        self._ok(L.viper_hip_qlinear_prequantized(Q4, p(wq[0]), p(wq[1]), 0, 64, nQ, H, p(self.xq), p(self.xs), 1,
                                                  p(self.q), None, st), "q")
        self._ok(L.viper_hip_qlinear_fused2_prequantized(Q4, p(wk[0]), p(wk[1]), p(wv[0]), p(wv[1]), 0, 64, nKV, H,
                                                         p(self.xq), p(self.xs), 1, p(self.k), p(self.v), st), "kv")
        self._ok(L.viper_hip_quantize_act(64, p(self.attn), 1, nQ, p(self.xq), p(self.xs), st), "quantize")
        self._ok(L.viper_hip_qlinear_prequantized(Q4, p(wo[0]), p(wo[1]), 0, 64, H, nQ, p(self.xq), p(self.xs), 1,
                                                  p(x), p(xin), st), "o")

    def mlp_half(self, l, fused=True):
        """Slot l's gate/up projections from rmsnorm(x), h = silu(gate) * up
        (left in self.gt), and the down projection of h added into x."""
        L, st = self.L, self.torch.cuda.current_stream().cuda_stream
        H, I = self.H, self.I
        p = lambda t: t.data_ptr()
        x = self.x
        wg, wu, wd = self.w[l % self.layers][4:]
        ln = self.ln[2 * (l % self.layers) + 1]
        if fused:
            self._m1_swiglu(2, p(x), p(ln), wg, wu, self.gt, eps=self.eps, st=st)
            self._m1(0, p(self.gt), None, [(wd, x)], residual=p(x), st=st)
            return
        self._ok(L.viper_hip_rmsnorm_quantize(p(x), p(ln), self.eps, 1, H, 64, p(self.xn), p(self.xq),
                                              p(self.xs), st), "rmsnorm_quantize")
        g = self.g if self.trace else self.gt   # the engine writes h over gate
        self._ok(L.viper_hip_qlinear_fused2_prequantized(Q4, p(wg[0]), p(wg[1]), p(wu[0]), p(wu[1]), 0, 64, I, H,
                                                         p(self.xq), p(self.xs), 1, p(g), p(self.ut), st),
                 "gate_up")
        self._ok(L.viper_hip_swiglu_quantize(p(g), p(self.ut), 1, I, 64, p(self.gt), p(self.xq), p(self.xs), st),
                 "swiglu_quantize")
        self._ok(L.viper_hip_qlinear_prequantized(Q4, p(wd[0]), p(wd[1]), 0, 64, H, I, p(self.xq), p(self.xs), 1,
                                                  p(x), p(x), st), "down")

    def head_step(self, fused=True):
        """Final rmsnorm of x (into self.xn), the bf16 LM head and the greedy token (fused: each
        logits row split over many workgroups, viper_hip_sampling_greedy_split)."""
        L, st = self.L, self.torch.cuda.current_stream().cuda_stream
        p = lambda t: t.data_ptr()
        self._ok(L.viper_hip_rmsnorm_quantize(p(self.x), p(self.final_ln), self.eps, 1, self.H, 64, p(self.xn),
                                              p(self.xq), p(self.xs), st), "final norm")
        self._ok(L.viper_hip_linear_bf16(p(self.head), p(self.xn), p(self.logits), 1, self.V, self.H, st), "lm_head")
        if fused:
            self._ok(L.viper_hip_sampling_greedy_split(p(self.logits), p(self.token), 1, self.V, p(self.greedy_ws),
                                                       self.greedy_ws.numel(), st), "greedy")
        else:
            self._ok(L.viper_hip_sampling_greedy(p(self.logits), p(self.token), 1, self.V, st), "greedy")

    def _prefetch(self, layer, workgroups):
        """Warm `layer`'s weight arena into the memory-side cache on the side stream, after the main
        stream's work so far has been issued (the event orders nothing on the main stream)."""
        torch = self.torch
        main = torch.cuda.current_stream()
        ev = torch.cuda.Event()
        ev.record(main)
        self.side.wait_event(ev)
        a = self.arenas[layer]
        self._ok(self.L.viper_hip_prefetch(a.data_ptr(), a.numel(), workgroups, self.sink.data_ptr(),
                                           self.side.cuda_stream), "prefetch")

    def _step(self, fused, prefetch=0):
        torch = self.torch
        slots = self.layers * self.passes
        if prefetch:
            if self.side is None:
                self.side = torch.cuda.Stream()
            self.side.wait_stream(torch.cuda.current_stream())
        for l in range(slots):
            if prefetch and l + 1 < slots:
                self._prefetch((l + 1) % self.layers, prefetch)
            self.attention_half(l, fused)
            self.mlp_half(l, fused)
        if prefetch:
            torch.cuda.current_stream().wait_stream(self.side)
        self.head_step(fused)

    def step_fused(self, prefetch=0):
        """One decode step, 4 launches per slot (producers folded, q/k/v together).  prefetch > 0:
        while slot s runs, a second stream warms slot s + 1's weights into the memory-side cache with
        that many workgroups (viper_hip_prefetch); the results are the same bit for bit."""
        self._step(True, prefetch)

    def step(self):
        """One decode step of the linear path, reference launch sequence."""
        self._step(False)
