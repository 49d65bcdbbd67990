"""Sequential GPTQ calibration of a Hugging Face Llama model into precomputed INT4 codes for the decode runtime.

The procedure of runtime/gptq.py:27-107 of the reference, on whatever device the HF model lives on:
  * the inputs of decoder layer 0 (and the keyword arguments the model passes to every layer: rotary embeddings,
    mask, positions) are captured from the calibration windows;
  * layer by layer, forward hooks accumulate the input Hessian H = sum x^T x of each projection group -- q/k/v share
    one input (one GPTQ call on the stacked [q; k; v] rows, which equals three calls since rows are independent),
    gate/up share one, o and down have their own -- and ``runtime.quant.quantize_gptq`` quantizes with 2 H / n;
  * the dequantized weights are written back into the layer before its outputs are recomputed as the next layer's
    inputs, so every layer is calibrated on the outputs of the already-quantized layers before it;
  * the LM head is calibrated last on the final-norm outputs; the HF model's weights are restored afterwards.

Output keys are those the runtime's ``DecodeConfig(quant="pre", qparams=...)`` reads: "layers.{i}.{qkv,o,gu,down}"
and "lm_head" -> (q uint8 [N, K], scale fp16 [N, K/G], zero fp16 [N, K/G]), on the CPU.

Calibration windows are the caller's token id tensors (the reference draws WikiText-2 windows through a dataset
download, runtime/gptq.py:17-24, which is not available offline): any local text tokenized, or random tokens.
"""
import time

import torch

from .quant import quantize_gptq


def dequantize(q, scale, zero, group):
    """fp16 [N, K] = fp16((q - zero) * scale) with one rounding (runtime/quant.py:93-97)."""
    N, K = q.shape
    qf = q.float().reshape(N, K // group, group)
    return ((qf - zero.float()[..., None]) * scale.float()[..., None]).reshape(N, K).half()


def random_windows(vocab, n=32, L=128, seed=0, bos=1):
    """n synthetic calibration windows of L token ids (bos first), for models without a local corpus."""
    g = torch.Generator().manual_seed(seed)
    return [torch.cat([torch.tensor([bos]), torch.randint(2, vocab, (L - 1,), generator=g)]) for _ in range(n)]


class _Captured(Exception):
    pass


@torch.no_grad()
def calibrate(hf, windows, group=128, clip=False, lm_head=True, log=print):
    """hf: a transformers LlamaForCausalLM (eval mode); windows: list of int64 token id tensors [L]. Returns the
    precomputed codes per projection (see the module docstring)."""
    dev = next(hf.parameters()).device
    layers = hf.model.layers
    inps, kw = [], {}
    first = layers[0]

    class Catcher(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.m = m

        def forward(self, hidden_states, *args, **kwargs):
            inps.append(hidden_states)
            kw.update(kwargs)
            raise _Captured

    layers[0] = Catcher(first)
    try:
        for w in windows:
            try:
                hf.model(w[None].to(dev), use_cache=False)
            except _Captured:
                pass
    finally:
        layers[0] = first
    kw = {k: v for k, v in kw.items() if k not in ("past_key_values", "past_key_value", "use_cache")}

    def run(layer, x):
        o = layer(x, **kw)
        return o[0] if isinstance(o, tuple) else o

    saved, out = {}, {}
    t0 = time.time()
    try:
        for i, layer in enumerate(layers):
            a, m = layer.self_attn, layer.mlp
            targets = {"qkv": (a.q_proj, [a.q_proj, a.k_proj, a.v_proj]), "o": (a.o_proj, [a.o_proj]),
                       "gu": (m.gate_proj, [m.gate_proj, m.up_proj]), "down": (m.down_proj, [m.down_proj])}
            H = {k: None for k in targets}
            cnt = {k: 0 for k in targets}

            def hook(key):
                def f(mod, args, _out):
                    x = args[0].reshape(-1, args[0].shape[-1]).float()
                    H[key] = x.t() @ x if H[key] is None else H[key] + x.t() @ x
                    cnt[key] += x.shape[0]
                return f

            hs = [mod.register_forward_hook(hook(k)) for k, (mod, _) in targets.items()]
            try:
                for x in inps:
                    run(layer, x)
            finally:
                for h in hs:
                    h.remove()
            for key, (_, mods) in targets.items():
                W = torch.cat([mm.weight.data for mm in mods], 0)
                q, s, z = quantize_gptq(W, 2 * H[key] / cnt[key], group, clip=clip)
                out[f"layers.{i}.{key}"] = (q.cpu(), s.cpu(), z.cpu())
                deq = dequantize(q, s, z, group)
                r = 0
                for mm in mods:
                    saved[id(mm)] = (mm, mm.weight.data.cpu().clone())
                    mm.weight.data.copy_(deq[r:r + mm.weight.shape[0]])
                    r += mm.weight.shape[0]
            del H
            inps = [run(layer, x) for x in inps]     # the next layer sees this layer's quantized outputs
            log(f"gptq layer {i}: {time.time() - t0:.1f}s")
        if lm_head:
            Hh, c = None, 0
            for x in inps:
                y = hf.model.norm(x).reshape(-1, x.shape[-1]).float()
                Hh = y.t() @ y if Hh is None else Hh + y.t() @ y
                c += y.shape[0]
            q, s, z = quantize_gptq(hf.lm_head.weight.data, 2 * Hh / c, group, clip=clip)
            out["lm_head"] = (q.cpu(), s.cpu(), z.cpu())
    finally:
        for mm, w in saved.values():                 # restore the model's own weights
            mm.weight.data.copy_(w.to(dev))
    log(f"gptq done: {time.time() - t0:.1f}s, {len(out)} matrices")
    return out
