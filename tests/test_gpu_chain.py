"""GPU tests of the chained launch (stark_qmm_encode_chain): one Qwen3-8B
layer's o -> gate/up -> down (three K slices) -> next q/k/v products in one
persistent launch, handing rows over through tagged words, against the same
products issued as separate launches (stark_qmm_encode_many and
stark_qmm_encode_many_prologue): every row must be the same bits, with the
tags the chain was told to write. Then the whole decode stand-in in its
chained form against the fused form (tokens, logits, residual row and KV
rows bit-identical), eager and as graph replays."""
import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu

H, I, QD, KD = 4096, 12288, 4096, 1024


@pytest.fixture(scope="module")
def D():
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from stark_amd import decode
    return decode


def _layer(D, seed):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)

    def qmat(n, k):
        codes, s, b = D.quantize_affine_gpu(torch.randn(n, k, generator=gen, device="cuda") * 0.02, 4, 64)
        return dict(n=n, k=k, bits=4, codes=codes, scales=s, biases=b)

    def norm_w(n):
        return (1.0 + 0.05 * torch.randn(n, generator=gen, device="cuda")).to(torch.bfloat16)

    L = dict(q=qmat(QD, H), k=qmat(KD, H), v=qmat(KD, H), o=qmat(H, QD), gate=qmat(I, H), up=qmat(I, H),
             down=qmat(H, I), mlp_norm=norm_w(H), next_norm=norm_w(H))
    x0 = torch.randn(H, generator=gen, device="cuda").to(torch.bfloat16)
    attn = torch.randn(QD, generator=gen, device="cuda").to(torch.bfloat16)
    return L, x0, attn


def _args(Q, mat, a, d, accumulate=False):
    return Q.MatmulArguments(
        a=a, m=1, n=mat["n"], k=mat["k"], d=d,
        b=Q.QuantizedB(codes=mat["codes"], scales=mat["scales"], correction_data=mat["biases"], mode=Q.MODE_U4,
                       group_size=64, params=Q.QuantParams(Q.GROUP_OUTPUT, mat["n"], mat["k"] // 64)),
        d_transform=Q.MatmulDOps(accumulate=accumulate))


def _separate(Q, L, x0, attn, eps=1e-6):
    """The layer as four launches (the fused decoder's form)."""
    K = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    x = x0.clone()
    g, u = torch.empty(I, dtype=torch.bfloat16, device="cuda"), torch.empty(I, dtype=torch.bfloat16, device="cuda")
    q, k, v = (torch.empty(n, dtype=torch.bfloat16, device="cuda") for n in (QD, KD, KD))
    K.encode_many([_args(Q, L["o"], attn, x, accumulate=True)])
    x1 = x.clone()
    K.encode_many_prologue([_args(Q, L["gate"], x, g), _args(Q, L["up"], x, u)], Q.PROLOGUE_RMS_NORM,
                           L["mlp_norm"], eps)
    K.encode_many_prologue([_args(Q, L["down"], g, x, accumulate=True)], Q.PROLOGUE_SILU_GATE, u)
    K.encode_many_prologue([_args(Q, L["q"], x, q), _args(Q, L["k"], x, k), _args(Q, L["v"], x, v)],
                           Q.PROLOGUE_RMS_NORM, L["next_norm"], eps)
    torch.cuda.synchronize()
    return dict(x1=x1, g=g, u=u, x=x, q=q, k=k, v=v)


def _chain_products(Q, L, xt, gt, ut, attn, q, k, v, tags, eps=1e-6, slices=3):
    to, tgu, td = tags
    CP = Q.ChainProduct
    return [CP(_args(Q, L["o"], attn, xt, accumulate=True), 0, out_tag=to),
            CP(_args(Q, L["gate"], xt, gt), 1, Q.PROLOGUE_RMS_NORM, L["mlp_norm"], eps, in_tag=to, out_tag=tgu),
            CP(_args(Q, L["up"], xt, ut), 1, Q.PROLOGUE_RMS_NORM, L["mlp_norm"], eps, in_tag=to, out_tag=tgu),
            CP(_args(Q, L["down"], gt, xt, accumulate=True), 2, Q.PROLOGUE_SILU_GATE, ut, in_tag=tgu, out_tag=td,
               acc_tag=to, k_slices=slices, part_tag=td),
            CP(_args(Q, L["q"], xt, q), 3, Q.PROLOGUE_RMS_NORM, L["next_norm"], eps, in_tag=td),
            CP(_args(Q, L["k"], xt, k), 3, Q.PROLOGUE_RMS_NORM, L["next_norm"], eps, in_tag=td),
            CP(_args(Q, L["v"], xt, v), 3, Q.PROLOGUE_RMS_NORM, L["next_norm"], eps, in_tag=td)]


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_chain_layer_matches_separate_launches(qmm, D):
    Q = qmm
    L, x0, attn = _layer(D, 5)
    want = _separate(Q, L, x0, attn)
    K = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    tags = (2, 3, 4)
    xt = Q.tag_rows(x0, 77)
    gt, ut = torch.zeros(I, dtype=torch.int32, device="cuda"), torch.zeros(I, dtype=torch.int32, device="cuda")
    q, k, v = (torch.zeros(n, dtype=torch.bfloat16, device="cuda") for n in (QD, KD, KD))
    chain = K.prepare_chain(_chain_products(Q, L, xt, gt, ut, attn, q, k, v, tags))
    assert chain.workspace_bytes == 256 + 2 * H * 8
    ws = torch.zeros(chain.workspace_bytes // 8, dtype=torch.int64, device="cuda")
    seq = torch.zeros(1, dtype=torch.int32, device="cuda")
    for call in range(2):  # the second call with the tag parity flipped
        seq.fill_(call)
        flip = call << 15
        xt.copy_(Q.tag_rows(x0, 77 ^ flip))
        gt.zero_()
        ut.zero_()
        print(f"chain call {call}", flush=True)
        K.encode_chain(chain, ws, seq)
        torch.cuda.synchronize()
        assert int(ws[0].item()) == 0, "a chained wait gave up"
        xv, xtag = Q.untag_rows(xt)
        gv, gtag = Q.untag_rows(gt)
        uv, utag = Q.untag_rows(ut)
        assert torch.all(xtag == (4 ^ flip)) and torch.all(gtag == (3 ^ flip)) and torch.all(utag == (3 ^ flip))
        assert _same(gv, want["g"]) and _same(uv, want["u"])
        assert _same(xv, want["x"])
        for name, t in (("q", q), ("k", k), ("v", v)):
            assert _same(t, want[name]), name
        # partial slices carry the down tag (word 1 of the workspace onward)
        parts = ws[32:].view(2, H)
        assert torch.all((parts >> 32) & 0xffffffff == (4 ^ flip))


def test_chain_down_slices_plain_rows_match_single_launch(qmm, D):
    """The fused decoder's down product: three K slices of one chained launch
    on plain bf16 rows (SiLU-gate prologue, accumulate into the residual),
    against stark_qmm_encode_many_prologue's one launch: the same bits, on two
    calls with the tag parity flipped between them."""
    Q = qmm
    L, x0, attn = _layer(D, 8)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    g = torch.randn(I, generator=gen, device="cuda").to(torch.bfloat16)
    u = torch.randn(I, generator=gen, device="cuda").to(torch.bfloat16)
    K = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    want = x0.clone()
    K.encode_many_prologue([_args(Q, L["down"], g, want, accumulate=True)], Q.PROLOGUE_SILU_GATE, u)
    x = x0.clone()
    chain = K.prepare_chain([Q.ChainProduct(_args(Q, L["down"], g, x, accumulate=True), 0, Q.PROLOGUE_SILU_GATE, u,
                                            k_slices=3, part_tag=7)])
    ws = torch.zeros(chain.workspace_bytes // 8, dtype=torch.int64, device="cuda")
    seq = torch.zeros(1, dtype=torch.int32, device="cuda")
    for call in range(2):
        seq.fill_(call)
        x.copy_(x0)
        K.encode_chain(chain, ws, seq)
        torch.cuda.synchronize()
        assert int(ws[0].item()) == 0
        assert _same(x, want)


def test_chain_waits_on_stale_tags_give_up_and_flag(qmm, D):
    """A consumer whose tag never arrives (here: the o stage is told to write
    tag 2 but the gate/up stage waits for tag 9) gives up after its bounded
    wait and flags the workspace status; the launch still ends."""
    Q = qmm
    L, x0, attn = _layer(D, 6)
    K = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    xt = Q.tag_rows(x0, 77)
    gt, ut = torch.zeros(I, dtype=torch.int32, device="cuda"), torch.zeros(I, dtype=torch.int32, device="cuda")
    q, k, v = (torch.zeros(n, dtype=torch.bfloat16, device="cuda") for n in (QD, KD, KD))
    prods = _chain_products(Q, L, xt, gt, ut, attn, q, k, v, (2, 3, 4))[:3]
    prods[1].in_tag = prods[2].in_tag = 9
    chain = K.prepare_chain(prods)
    ws = torch.zeros(chain.workspace_bytes // 8, dtype=torch.int64, device="cuda")
    K.encode_chain(chain, ws)
    torch.cuda.synchronize()
    assert int(ws[0].item()) != 0


def test_chain_rejects(qmm, D):
    Q = qmm
    L, x0, attn = _layer(D, 7)
    K = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
    xt = Q.tag_rows(x0, 1)
    gt, ut = torch.zeros(I, dtype=torch.int32, device="cuda"), torch.zeros(I, dtype=torch.int32, device="cuda")
    q, k, v = (torch.zeros(n, dtype=torch.bfloat16, device="cuda") for n in (QD, KD, KD))
    base = lambda: _chain_products(Q, L, xt, gt, ut, attn, q, k, v, (2, 3, 4))
    p = base()
    p[3].part_tag = 0  # K slices need a partial-sum tag
    with pytest.raises(Q.MatmulError):
        K.prepare_chain(p)
    p = base()
    p[3].prologue = Q.PROLOGUE_RMS_NORM  # the RMS-norm prologue needs K == 4096
    p[3].prologue_data = L["mlp_norm"]
    with pytest.raises(Q.MatmulError):
        K.prepare_chain(p)
    p = base()
    p[1].stage = 5  # stages out of order
    with pytest.raises(Q.MatmulError):
        K.prepare_chain(p)
    p = base()
    p[0].out_tag = 0x8000  # tags are 1..0x7fff
    with pytest.raises(Q.MatmulError):
        K.prepare_chain(p)
    chain = K.prepare_chain(base())
    small = torch.zeros(4, dtype=torch.int64, device="cuda")
    with pytest.raises(Q.MatmulError):
        K.encode_chain(chain, small)


def _run(D, chain, steps, graph):
    cfg = D.Qwen3Config()
    m = D.Qwen3Decoder(cfg, capacity=4096 + 8, seed=31, chain=chain)
    m.fill_context(4096, seed=32)
    if graph:
        m.step()  # builds the schedules
        torch.cuda.synchronize()
        g = m.capture()
        for _ in range(steps - 1):
            g.replay()
    else:
        for _ in range(steps):
            m.step()
    torch.cuda.synchronize()
    x = D.qmm_untag(m.xt) if chain else m.x
    out = dict(logits=m.logits.clone(), x=x.clone(), hist=m.history[4096:4096 + steps].clone(),
               kv=[torch.cat([L["kcache"][:, 4096:4096 + steps], L["vcache"][:, 4096:4096 + steps]]).clone()
                   for L in m.layers],
               status=m.chain_status() if chain else 0)
    del m
    torch.cuda.empty_cache()
    return out


@pytest.mark.parametrize("graph", [False, True])
def test_chain_decoder_matches_fused_full_size(D, graph):
    """Three greedy tokens of the full-size decoder (36 layers, 4096-token
    context) in the chained and in the fused form: the same bits."""
    print(f"decoder chain vs fused, graph={graph}", flush=True)
    a = _run(D, True, 3, graph)
    b = _run(D, False, 3, graph)
    assert a["status"] == 0
    assert torch.equal(a["hist"], b["hist"])
    assert _same(a["x"], b["x"])
    assert torch.equal(a["logits"], b["logits"])
    for i, (ka, kb) in enumerate(zip(a["kv"], b["kv"])):
        assert _same(ka, kb), f"layer {i} KV rows differ"
