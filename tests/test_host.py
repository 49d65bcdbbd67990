"""CPU checks of the runtime's host logic: the byte model of the decode step (scope row a10) against the figures the
reference publishes for its configurations (plots/predictions.json of the reference, as recorded for BASELINE configs 4
and 5), the gate/up row interleave the SwiGLU epilogues rely on, and the committed attention policy table."""
import torch

from runtime.model import byte_model, deinterleave_halves, interleave_halves
from runtime.synth import LLAMA3_8B, TINYLLAMA


def test_byte_model_tinyllama_matches_reference_figures():
    """Config 4: TinyLlama, INT4 G128 body, fp16 LM head: 658,993,664 B per token at context 512, 693,596,672 at
    2048 (body 514,899,968; head 131,072,000; activations 1,460,736)."""
    b512, b2k = byte_model(TINYLLAMA, 512), byte_model(TINYLLAMA, 2048)
    assert b512["body"] == 514_899_968 and b512["lm_head"] == 131_072_000
    assert b512["activations"] == 1_460_736 and b512["embedding_row"] == 4096
    assert b512["total"] == 658_993_664 and b2k["total"] == 693_596_672


def test_byte_model_llama3_8b_matches_reference_figures():
    """Config 5: Llama-3-8B body 3,708,289,024 B, LM head INT4 279,085,056 or fp16 1,050,673,152, KV at 4096
    537,001,984; the byte rooflines at 8 TB/s are 1,766 (INT4 head) and 1,509 (fp16 head) tokens/s."""
    i4, f16 = byte_model(LLAMA3_8B, 4096, head="int4"), byte_model(LLAMA3_8B, 4096, head="fp16")
    assert i4["body"] == 3_708_289_024 and i4["kv"] == 537_001_984
    assert i4["lm_head"] == 279_085_056 and f16["lm_head"] == 1_050_673_152
    assert round(8e12 / i4["total"]) == 1766 and round(8e12 / f16["total"]) == 1509


def test_byte_model_fp16_weights_and_context_scaling():
    """fp16 projections cost 4 x the INT4 payload without the (scale, zero) words; each context token adds the K and
    V rows of every layer."""
    i4, f16 = byte_model(TINYLLAMA, 0), byte_model(TINYLLAMA, 0, weights="fp16")
    norms = TINYLLAMA.num_hidden_layers * 4 * TINYLLAMA.hidden_size
    sz = TINYLLAMA.num_hidden_layers * 4 * (2560 * 16 + 2048 * 16 + 11264 * 16 + 2048 * 44)
    assert f16["body"] - norms == 4 * (i4["body"] - norms - sz)
    row = TINYLLAMA.num_key_value_heads * (TINYLLAMA.hidden_size // TINYLLAMA.num_attention_heads) * 2
    assert byte_model(TINYLLAMA, 101)["kv"] - byte_model(TINYLLAMA, 100)["kv"] == 2 * row * TINYLLAMA.num_hidden_layers


def test_interleave_halves_round_trip_and_order():
    t = torch.arange(12 * 3).view(12, 3)
    il = interleave_halves(t)
    assert torch.equal(il[0::2], t[:6]) and torch.equal(il[1::2], t[6:])
    assert torch.equal(deinterleave_halves(il), t)


def test_gemv_byte_count_matches_oracle():
    """The runtime's per-GEMV byte count (the roofline's `bytes_per_launch`) equals the oracle's format-derived one."""
    from oracle import quant_ref as Q
    from runtime.autotune import gemv_bytes
    for N, K, G in ((4096, 14336, 128), (14336, 4096, 128), (5632, 2048, 128), (2560, 2048, 64), (32000, 2048, 256)):
        assert gemv_bytes(N, K, G) == Q.gemv_bytes(N, K, G)


def test_attention_policy_entries_are_launchable():
    """Every entry of the committed attention policy is one the C ABI accepts for its head dim: impl 1 (block kernel)
    or 3 (lean kernel, part size a multiple of 16 up to 512 at head dim 64 and 256 at 128, as
    dk_paged_attention's version-5 check requires), contexts increasing, the last entry open-ended."""
    import json
    from runtime.model import DecodeConfig, Model
    pol = json.load(open(DecodeConfig().attn_policy_path))
    for key, D in (("policy", 64), ("policy_d128", 128)):
        ents = pol[key]
        assert [e["max_ctx"] for e in ents] == sorted(e["max_ctx"] for e in ents) and ents[-1]["max_ctx"] >= 1 << 30
        for e in ents:
            assert e["impl"] in (1, 3) and e["part_size"] > 0, e
            if e["impl"] == 3:
                assert e["part_size"] % 16 == 0 and e["part_size"] <= (256 if D == 128 else 512), e
        # the lookup picks the entry tuned at the largest context <= the cap
        for e in ents[:-1]:
            assert Model._policy_entry_of(pol, D, e["max_ctx"]) == e


def test_rope_theta_from_hf_configs():
    """The RoPE base comes from the config whichever way transformers stores it: the rope_theta attribute (4.x) or
    the rope_parameters dict (5.x, which has no attribute: reading only the attribute, as the reference's
    runtime/model.py:121 does, would rotate a Llama-3 config with base 10000 instead of 500000). Scaled RoPE types
    are refused instead of computed with the wrong frequencies."""
    import types
    import pytest
    from runtime.model import rope_theta_of
    assert rope_theta_of(types.SimpleNamespace(rope_theta=500000.0)) == 500000.0
    assert rope_theta_of(types.SimpleNamespace(rope_parameters={"rope_theta": 500000.0, "rope_type": "default"})) == 5e5
    assert rope_theta_of(types.SimpleNamespace(rope_scaling=None)) == 10000.0
    assert rope_theta_of(LLAMA3_8B) == 500000.0 and rope_theta_of(TINYLLAMA) == 10000.0
    with pytest.raises(NotImplementedError, match="llama3"):
        rope_theta_of(types.SimpleNamespace(rope_parameters={"rope_theta": 5e5, "rope_type": "llama3", "factor": 8.0}))
    try:
        from transformers import LlamaConfig
    except ImportError:
        return
    assert rope_theta_of(LlamaConfig(rope_theta=500000.0)) == 500000.0
    assert rope_theta_of(LlamaConfig()) == 10000.0
