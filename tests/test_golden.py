"""The oracle against vectors written by the reference's own code (tests/golden/make_golden.py runs runtime/quant.py
and runtime/model.py backend="ref" of the reference in the build container; only the outputs are committed).

* RTN quantize + pack at BASELINE config 1 scale: SHA-256 of the packed words and of the scale/zero halves, plus an
  edge matrix (all-zero group -> zero point -0.0, constant groups -> clamped zero points) in full.
* The decode step composition (runtime/model.py:216-233 over reference/ref_ops.py, INT4 G128 weights and LM head) on
  a tiny Llama: teacher-forced fp16 logits and greedy tokens."""
import hashlib
import json
import pathlib

import numpy as np
import torch

from oracle import quant_ref as Q
from oracle.decode_ref import RefDecoder

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _load_maker():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", GOLD / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_oracle_quantizer_matches_reference_at_config1_scale():
    mg = _load_maker()
    g = json.load(open(GOLD / "quant_cfg1.json"))
    q, s, z = Q.quantize(mg.cfg1_weight().numpy(), 128)
    packed, sz = Q.pack(q), Q.pack_scale_zero(s, z)
    assert packed[:2].astype(np.int64).tolist() == g["cfg1"]["packed_rows01"]
    assert sz[:2].view(np.uint16).astype(int).tolist() == g["cfg1"]["sz_rows01_bits"]
    assert _sha(packed) == g["cfg1"]["packed_sha256"] and _sha(sz) == g["cfg1"]["sz_sha256"]
    qe, se, ze = Q.quantize(mg.edge_weight().numpy(), 128)
    assert Q.pack(qe).astype(np.int64).tolist() == g["edge"]["packed"]
    assert Q.pack_scale_zero(se, ze).view(np.uint16).astype(int).tolist() == g["edge"]["sz_bits"]
    assert g["edge"]["sz_bits"][0][0][1] == 0x8000          # the all-zero group's zero point is fp16 -0.0


def tiny_oracle_weights(mg):
    """Fused, INT4-G128-quantized and dequantized weights of the tiny model, as the reference's Linear builds them
    (runtime/model.py:98-110, QuantLinear keep_ref)."""
    sd = mg.tiny_state_dict()
    c = mg.Cfg(mg.TINY)

    def deq(w):
        q, s, z = Q.quantize(w.numpy(), 128)
        return torch.from_numpy(Q.dequantize(q, s, z, 128))

    layers = []
    for i in range(c.num_hidden_layers):
        p = f"model.layers.{i}."
        layers.append({
            "ln1": sd[p + "input_layernorm.weight"], "ln2": sd[p + "post_attention_layernorm.weight"],
            "qkv": deq(torch.cat([sd[p + "self_attn.q_proj.weight"], sd[p + "self_attn.k_proj.weight"],
                                  sd[p + "self_attn.v_proj.weight"]])),
            "o": deq(sd[p + "self_attn.o_proj.weight"]),
            "gu": deq(torch.cat([sd[p + "mlp.gate_proj.weight"], sd[p + "mlp.up_proj.weight"]])),
            "down": deq(sd[p + "mlp.down_proj.weight"])})
    return {"emb": sd["model.embed_tokens.weight"], "norm_f": sd["model.norm.weight"],
            "lm_head": deq(sd["lm_head.weight"]), "layers": layers}, c


def test_oracle_decode_matches_reference_backend_ref():
    mg = _load_maker()
    gold = np.load(GOLD / "decode_tiny.npz")
    w, c = tiny_oracle_weights(mg)
    dec = RefDecoder(w, c, max_ctx=64, page=16, block_table=torch.from_numpy(gold["bt"]))
    logits = torch.stack([dec.step(int(t), p)[0] for p, t in enumerate(gold["tokens"])])
    want = torch.from_numpy(gold["logits"])
    err = (logits.float() - want.float()).abs().max() / want.float().abs().max()
    assert err <= 1e-3, float(err)                                     # same fp16 rounding points; sum order aside
    assert torch.equal(logits.float().argmax(-1), want.float().argmax(-1))
