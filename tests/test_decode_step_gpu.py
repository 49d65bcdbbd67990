"""Persistent decode step (dk_decode_step): one launch per token must give the decode step of the multi-launch path
(runtime/model.py:216-233 composition: qkv with the fused norm, RoPE + append + split attention + combine, o, gate|up
with the norm and the SwiGLU epilogue, down, the head, argmax + advance) and the CPU oracle decoder.

Bars: logits within 5e-3 (normwise) of the multi-launch step, which computes the same rounding points in a different
summation order; KV cache within 5e-3; 2e-2 and identical greedy tokens against the oracle decoder (the decode-step
bar of the smoke test); the sync words back at zero after every step; nothing touched when *pos is out of range.
"""
import pytest
import torch

from helpers import DEV, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime import ext
    return ext.load()


def _models(shape, max_ctx, seed=3, **kw):
    from runtime.model import DecodeConfig, Model
    from runtime.synth import SyntheticLlama
    sd = SyntheticLlama(shape, seed=seed, device=DEV, std=0.05, norm_std=0.1)
    multi = Model(sd, shape, DecodeConfig(max_ctx=max_ctx, device=DEV, **kw))
    pers = Model(sd, shape, DecodeConfig(max_ctx=max_ctx, device=DEV, persistent=True, **kw))
    assert torch.equal(multi.bt.cpu(), pers.bt.cpu())
    return multi, pers


def _tokens(n, V, seed=0):
    return torch.randint(0, V, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


# (shape, teacher-forced tokens): head dim 64 with GQA 2 and 4, head dim 128; contexts below one split (128 tokens)
# and across several splits (combine phase)
CASES = [
    ((256, 2, 4, 2, 512, 1000), 40),
    ((256, 2, 4, 2, 512, 1000), 300),
    ((512, 3, 8, 2, 1024, 700), 150),
    ((512, 2, 4, 2, 1024, 1000), 270),
]


@pytest.mark.parametrize("shape_t,n", CASES)
def test_persistent_step_matches_multi_launch_step(K, shape_t, n):
    from runtime.synth import LlamaShape
    shape = LlamaShape(*shape_t)
    print(f"persistent vs multi-launch: shape {shape_t} tokens {n}", flush=True)
    multi, pers = _models(shape, max_ctx=512)
    for m in (multi, pers):
        m.prepare(512)
        m.reset(0)
    toks = _tokens(n, shape.vocab_size)
    a = multi.teacher_force(toks, collect_logits=True)
    b = pers.teacher_force(toks, collect_logits=True)
    torch.cuda.synchronize()
    for i in sorted({0, 1, n // 2, n - 2, n - 1}):
        assert_close(b[i], a[i], 5e-3, f"logits at position {i}")
    # the appended K / V rows of every layer (positions 0..n-1 through the block table)
    rows = multi.bt[: (n + 15) // 16].long()
    assert_close(pers.kv[:, :, rows], multi.kv[:, :, rows], 5e-3, "KV cache")
    assert int(pers.pos.item()) == n
    assert int(pers.step_sync.abs().sum().item()) == 0, "sync words must be left zero"
    assert pers.step_status() == 0


def test_persistent_step_eager_equals_graph(K):
    """The step launched eagerly and replayed from the captured graph gives the same tokens and logits."""
    from runtime.synth import LlamaShape
    shape = LlamaShape(256, 2, 4, 2, 512, 1000)
    _, pers = _models(shape, max_ctx=256)
    toks = _tokens(20, shape.vocab_size, seed=1)
    pers.prepare(256)
    pers.reset(0)
    g = pers.teacher_force(toks, collect_logits=True).clone()
    pers.reset(0)
    e = pers.teacher_force(toks, use_graph=False, collect_logits=True)
    assert torch.equal(g, e)


def test_persistent_step_against_oracle(K):
    """Greedy decoding through the persistent step against the CPU oracle decoder (oracle/decode_ref.py)."""
    import __graft_entry__ as ge
    from oracle.decode_ref import RefDecoder
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(256, 2, 4, 2, 512, 1000)
    m = Model(SyntheticLlama(shape, seed=1, device=DEV, std=0.05), shape,
              DecodeConfig(max_ctx=64, device=DEV, persistent=True))
    m.prepare(64)
    ref = RefDecoder(ge._ref_weights(m, shape), shape, max_ctx=64, page=16, block_table=m.bt.cpu())
    m.reset(0)
    tok = 5
    for p in range(12):
        m.tok.fill_(tok)
        m.run_step()
        lr, _ = ref.step(tok, p)
        assert_close(m.logits, lr, 2e-2, f"step {p}")
        nxt = int(m.tok.item())
        assert nxt == int(torch.argmax(m.logits.float().cpu())), p
        assert nxt == int(torch.argmax(lr.float())), p
        tok = nxt


@pytest.mark.parametrize("head", ["fp16", "int4"])
def test_persistent_step_real_widths(K, head):
    """TinyLlama widths (hidden 2048, 32 q / 4 kv heads, SwiGLU 5632, vocab 32000) on 2 layers at a context spanning
    five splits, fp16 and INT4 heads."""
    from runtime.synth import LlamaShape
    shape = LlamaShape(2048, 2, 32, 4, 5632, 32000)
    print(f"tinyllama widths, {head} head", flush=True)
    multi, pers = _models(shape, max_ctx=1024, lm_head=head)
    for m in (multi, pers):
        m.prepare(1024)
        m.reset(0)
    toks = _tokens(600, shape.vocab_size, seed=2)
    a = multi.teacher_force(toks, collect_logits=True)
    b = pers.teacher_force(toks, collect_logits=True)
    for i in (0, 127, 128, 599):
        assert_close(b[i], a[i], 5e-3, f"logits at position {i}")
    assert torch.equal(pers.tok.cpu(), multi.tok.cpu())


def test_persistent_step_llama3_widths(K):
    """Llama-3-8B widths (hidden 4096, 32 q / 8 kv heads of 128 dims, SwiGLU 14336) on 2 layers, INT4 head over a
    32000-token vocabulary, context across splits."""
    from runtime.synth import LlamaShape
    shape = LlamaShape(4096, 2, 32, 8, 14336, 32000, 1e-5, 500000.0)
    print("llama-3 widths", flush=True)
    multi, pers = _models(shape, max_ctx=512, lm_head="int4")
    for m in (multi, pers):
        m.prepare(512)
        m.reset(0)
    toks = _tokens(200, shape.vocab_size, seed=4)
    a = multi.teacher_force(toks, collect_logits=True)
    b = pers.teacher_force(toks, collect_logits=True)
    for i in (0, 128, 199):
        assert_close(b[i], a[i], 5e-3, f"logits at position {i}")


def test_persistent_step_position_out_of_range(K):
    """*pos outside [0, max_pos): the launch touches nothing (tok, pos, logits, cache unchanged)."""
    from runtime.synth import LlamaShape
    shape = LlamaShape(256, 2, 4, 2, 512, 1000)
    _, pers = _models(shape, max_ctx=64)
    pers.prepare(64)
    pers.logits.fill_(1.5)
    pers.tok.fill_(7)
    bad = pers.cos.shape[0]
    pers.pos.fill_(bad)
    kv = pers.kv.clone()
    pers.step()
    torch.cuda.synchronize()
    assert int(pers.pos.item()) == bad and int(pers.tok.item()) == 7
    assert torch.equal(pers.kv, kv)
    assert bool((pers.logits == 1.5).all())
    assert int(pers.step_sync.abs().sum().item()) == 0
