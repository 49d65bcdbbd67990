"""Sequential GPTQ calibration of a Hugging Face Llama model into precomputed INT4 codes for the decode runtime.

Behaviour of runtime/gptq.py:27-107 of the reference (layer by layer; each layer calibrated on the outputs of the
already-quantized layers before it; q/k/v and gate/up quantized as one stacked matrix each because they read the same
input; the LM head last, on the final-norm outputs; the model's own weights restored at the end). The structure here:

  * ``_LayerInputs``: a forward pre-hook on decoder layer 0 records the hidden states of every calibration window
    together with the keyword arguments the model hands each layer (rotary embeddings, mask, positions) and stops the
    forward there;
  * ``_HessianSet``: forward pre-hooks on the first projection of each input group (q_proj, o_proj, gate_proj,
    down_proj) accumulate X^T X of that group's input in float64 while the layer runs over the windows; the Hessian
    GPTQ receives is 2 X^T X / n in float32;
  * ``_Snapshot``: the original weight of every projection the calibration overwrites, restored on exit (also when
    an exception ends the calibration early).

Output keys are those ``DecodeConfig(quant="pre", qparams=...)`` reads: "layers.{i}.{qkv,o,gu,down}" and "lm_head" ->
(q uint8 [N, K], scale fp16 [N, K/G], zero fp16 [N, K/G]) on the CPU.

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


class _StopForward(Exception):
    """Raised by the layer-0 pre-hook once the layer's inputs are recorded."""


class _LayerInputs:
    """Hidden states entering decoder layer 0 for each window, and the per-layer keyword arguments."""

    def __init__(self, hf, windows):
        self.states, self.kwargs = [], {}
        dev = next(hf.parameters()).device

        def grab(_mod, args, kwargs):
            self.states.append(args[0] if args else kwargs["hidden_states"])
            self.kwargs.update({k: v for k, v in kwargs.items() if k != "hidden_states"})
            raise _StopForward

        handle = hf.model.layers[0].register_forward_pre_hook(grab, with_kwargs=True)
        try:
            for w in windows:
                try:
                    hf.model(w[None].to(dev), use_cache=False)
                except _StopForward:
                    pass
        finally:
            handle.remove()
        for k in ("past_key_values", "past_key_value", "use_cache"):   # no cache inside the calibration
            self.kwargs.pop(k, None)

    def through(self, layer):
        """Replace the stored states by the layer's outputs on them."""
        outs = []
        for x in self.states:
            y = layer(x, **self.kwargs)
            outs.append(y[0] if isinstance(y, tuple) else y)
        self.states = outs


class _HessianSet:
    """Per input group: sum over calibration tokens of x x^T (float64) and the token count, fed by pre-hooks."""

    def __init__(self, owners):
        self.sums, self.count, self.handles = {}, {}, []
        for key, mod in owners.items():
            self.handles.append(mod.register_forward_pre_hook(self._hook(key)))

    def _hook(self, key):
        def f(_mod, args):
            x = args[0].reshape(-1, args[0].shape[-1]).to(torch.float64)
            prev = self.sums.get(key)
            self.sums[key] = x.t() @ x if prev is None else prev.addmm_(x.t(), x)
            self.count[key] = self.count.get(key, 0) + x.shape[0]
        return f

    def close(self):
        for h in self.handles:
            h.remove()
        self.handles = []

    def hessian(self, key):
        return (2.0 * self.sums[key] / self.count[key]).float()


class _Snapshot:
    """Context manager: remembers each weight the first time it is overwritten and puts every one back on exit."""

    def __init__(self):
        self.kept = []
        self.seen = set()

    def overwrite(self, mod, value):
        if id(mod) not in self.seen:
            self.seen.add(id(mod))
            self.kept.append((mod, mod.weight.data.clone()))
        mod.weight.data.copy_(value)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        for mod, w in self.kept:
            mod.weight.data.copy_(w)
        return False


def _groups(layer):
    """Input group -> (projection whose input is the group's input, projections stacked into one GPTQ matrix)."""
    a, m = layer.self_attn, layer.mlp
    return {"qkv": (a.q_proj, (a.q_proj, a.k_proj, a.v_proj)), "o": (a.o_proj, (a.o_proj,)),
            "gu": (m.gate_proj, (m.gate_proj, m.up_proj)), "down": (m.down_proj, (m.down_proj,))}


@torch.no_grad()
def calibrate(hf, windows, group=128, clip=False, lm_head=True, log=print):
    """hf: a transformers LlamaForCausalLM (eval mode); windows: list of int64 token id tensors [L]. Returns the
    precomputed codes per projection (see the module docstring)."""
    t0 = time.time()
    inputs = _LayerInputs(hf, windows)
    out = {}
    with _Snapshot() as snap:
        for i, layer in enumerate(hf.model.layers):
            groups = _groups(layer)
            hs = _HessianSet({key: owner for key, (owner, _) in groups.items()})
            try:
                for x in inputs.states:
                    layer(x, **inputs.kwargs)
            finally:
                hs.close()
            for key, (_, mods) in groups.items():
                stacked = torch.cat([mod.weight.data for mod in mods], 0)
                q, s, z = quantize_gptq(stacked, hs.hessian(key), group, clip=clip)
                out[f"layers.{i}.{key}"] = (q.cpu(), s.cpu(), z.cpu())
                for mod, part in zip(mods, dequantize(q, s, z, group).split([m.weight.shape[0] for m in mods])):
                    snap.overwrite(mod, part)
            inputs.through(layer)          # the next layer sees this layer's quantized outputs
            log(f"gptq layer {i}: {time.time() - t0:.1f}s")
        if lm_head:
            normed = [hf.model.norm(x).reshape(-1, x.shape[-1]).to(torch.float64) for x in inputs.states]
            acc = sum(y.t() @ y for y in normed)
            n = sum(y.shape[0] for y in normed)
            q, s, z = quantize_gptq(hf.lm_head.weight.data, (2.0 * acc / n).float(), group, clip=clip)
            out["lm_head"] = (q.cpu(), s.cpu(), z.cpu())
    log(f"gptq done: {time.time() - t0:.1f}s, {len(out)} matrices")
    return out
