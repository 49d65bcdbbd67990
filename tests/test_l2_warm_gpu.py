"""GPU checks of dk_paged_attention_warm, the attention launch whose spare workgroups read the weights of the GEMVs
that follow it into L2: it writes nothing beyond what dk_paged_attention (split_only 0) or dk_paged_attention_split
(split_only 1) write, so its output, partials and cache are those calls' bit for bit (the reference's op is
kernels/paged_attention.cu:429-461). Cases: the lean and the block split kernel, head dims 64 and 128, one live split
and several, spare splits, one and two GEMVs (row tiles that do and do not divide N, K up to 5632), warm-up
workgroup counts that do and do not fill whole grid rows; and the decode step with the warm-up against the step
without it (logits and cache identical over 40 teacher-forced tokens)."""
import pytest
import torch

from helpers import DEV, gen, make_cache

pytestmark = pytest.mark.gpu
G = 128


@pytest.fixture(scope="module")
def K():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime import ext
    return ext.load()


def _gemv(N, Kd, seed, cfg):
    g = torch.Generator(device=DEV).manual_seed(seed)
    packed = torch.randint(-2**31, 2**31 - 1, (N, Kd // 8), generator=g, dtype=torch.int32, device=DEV)
    sz = torch.randn(N, Kd // G, 2, generator=g, device=DEV).half()
    return packed, sz, G, cfg


GEMVS = {"o": (2048, 2048, (4, 2, 4, 0)), "gu": (11264, 2048, (4, 4, 0, 2)), "odd": (1000, 5632, (4, 2, 3, 1)),
         "wide": (4096, 4096, (4, 2, 4, 2))}

# (D, n_q, n_kv, ctx, part size, spare splits, version, split_only, warm-up workgroups, GEMVs)
CASES = [(64, 32, 4, 500, 128, 0, 5, 1, 232, ("o", "gu")),
         (64, 32, 4, 500, 128, 1, 5, 0, 13, ("o",)),
         (64, 32, 4, 1, 64, 2, 5, 1, 64, ("odd",)),
         (128, 32, 8, 700, 256, 0, 5, 0, 120, ("wide",)),
         (128, 32, 8, 300, 64, 1, 2, 1, 57, ("o", "odd")),
         (64, 16, 2, 129, 32, 0, 3, 0, 8, ("gu",))]


@pytest.mark.parametrize("D,n_q,n_kv,ctx,PS,spare,version,split_only,wgs,names", CASES)
def test_warm_matches_plain_attention(K, D, n_q, n_kv, ctx, PS, spare, version, split_only, wgs, names):
    page = 16
    S = -(-ctx // PS) + spare
    print(f"l2 warm D{D} {n_q}/{n_kv} ctx {ctx} PS {PS} splits {S} v{version} split_only {split_only} wgs {wgs} "
          f"{names}", flush=True)
    kc, vc, bt = make_cache(ctx + spare * PS, n_kv, page, D=D, seed=ctx + D)
    q = torch.randn(n_q * D, generator=gen(ctx + 3)).half().to(DEV)
    kd, vd, btd = kc.to(DEV), vc.to(DEV), bt.to(DEV)
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=DEV)
    nxt = [_gemv(*GEMVS[n][:2], seed=i + 1, cfg=GEMVS[n][2]) for i, n in enumerate(names)]
    before = [(p.clone(), s.clone()) for p, s, _, _ in nxt]
    res = []
    for warm in (False, True):
        f32 = dict(dtype=torch.float32, device=DEV)
        o, m, l = (torch.full(sh, 7.0, **f32) for sh in ((n_q, S, D), (n_q, S), (n_q, S)))
        out = torch.full((n_q * D,), 3.0, dtype=torch.half, device=DEV)
        args = (q, kd, vd, btd, pos, PS, o, m, l, out, version)
        if warm:
            K.paged_attention_warm(*args, split_only, nxt, wgs)
        elif split_only:
            K.paged_attention_split(*args)
        else:
            K.paged_attention(*args)
        torch.cuda.synchronize()
        res.append((o, m, l, out))
    for a, b, what in zip(res[0], res[1], ("o_part", "m_part", "l_part", "out")):
        assert torch.equal(a, b), f"{what} differs with the warm-up"
    for (p, s, _, _), (p0, s0) in zip(nxt, before):
        assert torch.equal(p, p0) and torch.equal(s, s0), "the warm-up must not write the weights it reads"


@pytest.mark.parametrize("combine_in_o", [True, False])
def test_decode_step_with_warm_up(combine_in_o):
    """The decode step with the warm-up (DecodeConfig.l2_warm) gives the step without it bit for bit: logits of
    every teacher-forced token and the KV cache pages written; the warm-up path is really taken (GEMVs listed,
    spare workgroups)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runtime.model import DecodeConfig, Model
    from runtime.synth import LlamaShape, SyntheticLlama
    shape = LlamaShape(512, 2, 8, 2, 1024, 1000)
    print(f"l2 warm decode combine_in_o {combine_in_o}", flush=True)
    sd = SyntheticLlama(shape, seed=6, device=DEV, std=0.05, norm_std=0.1)
    ms = [Model(sd, shape, DecodeConfig(max_ctx=256, device=DEV, combine_in_o=combine_in_o, l2_warm=w))
          for w in (False, True)]
    for m in ms:
        m.prepare(64, part_size=16)
        m.reset(0)
    b = ms[1]
    assert b.l2_warm_next(0) and b.l2_warm_wgs() > 0 and b.attn_in_o == combine_in_o
    toks = torch.randint(0, shape.vocab_size, (40,), generator=torch.Generator().manual_seed(2)).tolist()
    la = ms[0].teacher_force(toks, collect_logits=True)
    lb = b.teacher_force(toks, collect_logits=True)
    for i, (x, y) in enumerate(zip(la, lb)):
        assert torch.equal(x, y), f"logits differ at position {i}"
    rows = ms[0].bt[: (40 + 15) // 16].long()
    assert torch.equal(ms[0].bt, b.bt)
    assert torch.equal(ms[0].kv[:, :, rows], b.kv[:, :, rows]), "kv cache differs"
