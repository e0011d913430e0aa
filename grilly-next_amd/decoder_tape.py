"""A decoder stack driven through the tape engine: the end-to-end backward workload.

Per layer (pre-LN):  n1 = LN(x);  qkv = n1 Wqkv^T + bqkv;  o = causal attention over the
fused qkv rows;  x2 = x + o Wo^T + bo;  n2 = LN(x2);  h = gate * GELU_tanh(up) with
gate = n2 Wg^T + bg, up = n2 Wu^T + bu;  x3 = x2 + h Wd^T + bd.
Embedding x0 = E[ids], final LN, tied LM head logits = LN(x_L) E^T, cross-entropy over the
vocabulary (scale 1/T).  bf16 weights and block activations, fp32 statistics and weight
gradients; the residual stream x (and so its gradient) is fp32: the norms read it in fp32 and
write bf16, each bf16 branch output is added into it in fp32.  Carried in bf16, the residual
gradient's rounding over the 12 layers reaches the LayerNorm gains' gradient (a sum that
cancels heavily) at a few percent; in fp32 it stays within the bf16 tolerance.

`Decoder.forward()` runs the forward on the GPU through this library's forward kernels
(untimed: gn_layernorm_fwd saving mean/rstd, gn_linear_fwd, gn_glu_linear_fwd saving the
gate/up caches, gn_attn_fwd saving the fp32 row logsumexp; torch only for the embedding
gather and the residual adds) and keeps every tensor the backward needs.  `Decoder.record(tape)`
records the nodes the reference's tape would hold for this model (Linear, LayerNorm,
FlashAttention2, Add, CrossEntropy; autograd.h:81-141) plus this build's FusedGLU and
Embedding nodes, with the saved-slot conventions of each handler.
"""
import torch

import grilly_bridge as gb
import grilly_core
import gn_bwd as gn


class Decoder:
    def __init__(self, layers=12, d=768, heads=12, ff=3072, vocab=32000, batch=8, seq=1024,
                 seed=5, device="cuda:0", glu_epilogue=True):
        self.L, self.d, self.H, self.ff, self.V = layers, d, heads, ff, vocab
        self.glu_epilogue = glu_epilogue
        self.B, self.S, self.T = batch, seq, batch * seq
        self.dev = torch.device(device)
        g = torch.Generator(device=self.dev)
        g.manual_seed(seed)
        bf = torch.bfloat16

        def w(*shape):
            return (torch.randn(*shape, device=self.dev, generator=g) * 0.02).to(bf).contiguous()

        def const(n, v):
            return torch.full((n,), float(v), device=self.dev, dtype=bf)

        self.E = w(vocab, d)
        self.layers = [dict(ln1_g=const(d, 1), ln1_b=const(d, 0), Wqkv=w(3 * d, d),
                            bqkv=const(3 * d, 0), Wo=w(d, d), bo=const(d, 0), ln2_g=const(d, 1),
                            ln2_b=const(d, 0), Wg=w(ff, d), Wu=w(ff, d), bg=const(ff, 0),
                            bu=const(ff, 0), Wd=w(d, ff), bd=const(d, 0))
                       for _ in range(layers)]
        self.lnf_g, self.lnf_b = const(d, 1), const(d, 0)
        ids = torch.randint(0, vocab, (batch, seq), device=self.dev, generator=g)
        self.ids = ids.reshape(-1).to(torch.int32).contiguous()
        self.tgt = torch.roll(ids, -1, dims=1).reshape(-1).to(torch.int32).contiguous()
        self.loss = torch.zeros(1, device=self.dev)
        self.acts = None

    # ------------------------------------------------------------------ forward (untimed)
    def forward(self):
        B, S, H, d, T = self.B, self.S, self.H, self.d, self.T
        D = d // H
        ws = gn.workspace(gn.attn_workspace_bytes(B, H, S, D, gn.BF16), self.dev)
        bf = torch.bfloat16
        x = self.E[self.ids.long()].float().contiguous()  # fp32 residual stream
        self.x0 = x
        acts = []
        for p in self.layers:
            a = {"x": x}
            a["n1"], a["m1"], a["r1"] = gn.layernorm_fwd(x, p["ln1_g"], p["ln1_b"], out_dtype=bf)
            a["qkv"] = gn.linear_fwd(a["n1"], p["Wqkv"], p["bqkv"])
            q, k, v = (t.contiguous() for t in a["qkv"].view(B, S, 3, H, D).permute(2, 0, 3, 1, 4))
            O, a["lse"] = gn.attn_fwd(q, k, v, causal=True, rope="none", ws=ws)
            a["o"] = O.permute(0, 2, 1, 3).reshape(T, d).contiguous()
            a["ao"] = gn.linear_fwd(a["o"], p["Wo"], p["bo"])
            a["x2"] = (x + a["ao"].float()).contiguous()
            a["n2"], a["m2"], a["r2"] = gn.layernorm_fwd(a["x2"], p["ln2_g"], p["ln2_b"], out_dtype=bf)
            a["gate"], a["up"], a["h"] = gn.glu_linear_fwd("geglu_up", a["n2"], p["Wg"], p["Wu"],
                                                           p["bg"], p["bu"])
            a["f"] = gn.linear_fwd(a["h"], p["Wd"], p["bd"])
            a["x3"] = (a["x2"] + a["f"].float()).contiguous()
            acts.append(a)
            x = a["x3"]
        self.nf, self.mf, self.rf = gn.layernorm_fwd(x, self.lnf_g, self.lnf_b, out_dtype=bf)
        self.logits = gn.linear_fwd(self.nf, self.E)
        self.acts = acts
        torch.cuda.synchronize()

    # ------------------------------------------------------------------ tape
    def record(self, tape):
        """Record the forward's nodes (the forward must have run); returns the loss node."""
        assert self.acts is not None, "run forward() first"
        op, t, P = grilly_core.OpType, gb.tref, (lambda x: x.data_ptr())
        B, S, H, d = self.B, self.S, self.H, self.d
        n = tape.record_op(op.Embedding, [t(self.ids)], [t(self.x0)], gb.embedding_params(self.V))
        tape.save_for_backward(n, [P(self.E)])
        for p, a in zip(self.layers, self.acts):
            n = tape.record_op(op.LayerNorm, [t(a["x"], True)], [t(a["n1"])], gb.layernorm_params())
            tape.save_for_backward(n, [P(p["ln1_g"]), P(p["ln1_b"]), P(a["m1"]), P(a["r1"])])
            n = tape.record_op(op.Linear, [t(a["n1"], True)], [t(a["qkv"])])
            tape.save_for_backward(n, [P(p["Wqkv"]), P(p["bqkv"])])
            qkv = gb.make_tensor_ref(P(a["qkv"]), (B, S, 3 * d), gb.DTYPE_BF16, True)
            o = gb.make_tensor_ref(P(a["o"]), (B, S, d), gb.DTYPE_BF16)
            n = tape.record_op(op.FlashAttention2, [qkv], [o],
                               gb.attention_params(causal=True, rope="none", fused_qkv_heads=H))
            tape.save_for_backward(n, [P(a["lse"])])
            n = tape.record_op(op.Linear, [t(a["o"], True)], [t(a["ao"])])
            tape.save_for_backward(n, [P(p["Wo"]), P(p["bo"])])
            tape.record_op(op.Add, [t(a["x"], True), t(a["ao"], True)], [t(a["x2"])])
            n = tape.record_op(op.LayerNorm, [t(a["x2"], True)], [t(a["n2"])], gb.layernorm_params())
            tape.save_for_backward(n, [P(p["ln2_g"]), P(p["ln2_b"]), P(a["m2"]), P(a["r2"])])
            n = tape.record_op(op.FusedGLU, [t(a["n2"], True)], [t(a["h"])],
                               gb.fused_glu_params("geglu_up"))
            tape.save_for_backward(n, [P(p["Wg"]), P(p["Wu"]), P(a["gate"]), P(a["up"]),
                                       P(p["bg"]), P(p["bu"])])
            n = tape.record_op(op.Linear, [t(a["h"], True)], [t(a["f"])])
            tape.save_for_backward(n, [P(p["Wd"]), P(p["bd"])])
            tape.record_op(op.Add, [t(a["x2"], True), t(a["f"], True)], [t(a["x3"])])
        last = self.acts[-1]["x3"]
        n = tape.record_op(op.LayerNorm, [t(last, True)], [t(self.nf)], gb.layernorm_params())
        tape.save_for_backward(n, [P(self.lnf_g), P(self.lnf_b), P(self.mf), P(self.rf)])
        n = tape.record_op(op.Linear, [t(self.nf, True)], [t(self.logits)])
        tape.save_for_backward(n, [P(self.E)])
        return tape.record_op(op.CrossEntropy, [t(self.logits, True), t(self.tgt)], [t(self.loss)],
                              gb.cross_entropy_params(1.0 / self.T))

    def backward_step(self, tape):
        """One end-to-end backward through the tape: begin, record, backward, end.  The tape
        runs with set_glu_epilogue(True): each down projection forms its GLU's local gradients
        in its input-gradient GEMM (the GLU output's gradient is not kept)."""
        tape.set_glu_epilogue(self.glu_epilogue)
        tape.begin()
        loss = self.record(tape)
        tape.backward(loss, 0)
        tape.end()

    def flops(self):
        """Backward GEMM + attention FLOPs (dX and dW of every projection, causal attention
        with the P recompute counted once: 5 products over half the score matrix)."""
        T, d, ff, V, S, H = self.T, self.d, self.ff, self.V, self.S, self.H
        per_layer = (2 * 2 * T * d * 3 * d + 2 * 2 * T * d * d + 2 * 2 * T * d * ff * 2
                     + 2 * 2 * T * ff * d + 5 * 2.0 * S * S * (d // H) * 0.5 * self.B * H)
        return self.L * per_layer + 2 * 2 * T * d * V

    def fwd_flops(self):
        """Forward GEMM + attention FLOPs: every projection once, causal attention as 2
        products over half the score matrix, the LM head."""
        T, d, ff, V, S, H = self.T, self.d, self.ff, self.V, self.S, self.H
        per_layer = (2 * T * d * 3 * d + 2 * T * d * d + 2 * T * d * ff * 2 + 2 * T * ff * d
                     + 2 * 2.0 * S * S * (d // H) * 0.5 * self.B * H)
        return self.L * per_layer + 2 * T * d * V
