"""GPU tests of the config-4 decode stand-in (libstark_decode + the quantized
products): each decode-step kernel against a plain torch fp32 restatement,
one whole token step of a small Qwen3-shaped decoder against a torch fp32
forward over the dequantized weights, and graph replay against eager steps
(bit-identical tokens, positions and caches)."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def D():
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from stark_amd import decode
    return decode


def _p(t):
    return C.c_void_p(t.data_ptr())


def _s():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _bf(t):
    return t.to(torch.bfloat16).float()


def _rms(x, w, eps):
    x = x.float()
    return _bf(_bf(x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)) * w.float())


def _rope(x, pos, theta, hd=128):
    i = torch.arange(hd // 2, device=x.device, dtype=torch.float64)
    ang = pos * theta ** (-2.0 * i / hd)
    c, s = torch.cos(ang).float(), torch.sin(ang).float()
    a, b = x[..., : hd // 2], x[..., hd // 2:]
    return torch.cat([a * c - b * s, b * c + a * s], -1)


def test_rms_norm(D):
    torch.manual_seed(0)
    for n in (256, 4096):
        x = torch.randn(n, device="cuda").to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(n, device="cuda")).to(torch.bfloat16)
        out = torch.empty_like(x)
        assert D.lib().stark_decode_rms_norm(_p(x), _p(w), _p(out), n, 1e-6, _s()) == 0
        want = _rms(x, w, 1e-6)
        torch.testing.assert_close(out.float(), want, rtol=1e-2, atol=1e-2)
    assert D.lib().stark_decode_rms_norm(_p(x), _p(w), _p(out), 100, 1e-6, _s()) == 1


def test_qk_norm_rope_writes_cache(D):
    torch.manual_seed(1)
    qh, kvh, cap, pos = 8, 2, 64, 37
    q = torch.randn(qh * 128, device="cuda").to(torch.bfloat16)
    k = torch.randn(kvh * 128, device="cuda").to(torch.bfloat16)
    v = torch.randn(kvh * 128, device="cuda").to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(128, device="cuda")).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, device="cuda")).to(torch.bfloat16)
    kc = torch.zeros(kvh, cap, 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    q0 = q.clone()
    assert D.lib().stark_decode_qk_norm_rope(_p(q), _p(k), _p(v), _p(qw), _p(kw), _p(kc), _p(vc), _p(p), qh, kvh,
                                             cap, 1e6, 1e-6, _s()) == 0
    wq = _rope(_rms(q0.view(qh, 128), qw, 1e-6), pos, 1e6)
    wk = _rope(_rms(k.view(kvh, 128), kw, 1e-6), pos, 1e6)
    torch.testing.assert_close(q.view(qh, 128).float(), wq, rtol=1e-2, atol=2e-2)
    torch.testing.assert_close(kc[:, pos].float(), wk, rtol=1e-2, atol=2e-2)
    assert torch.equal(vc[:, pos], v.view(kvh, 128))
    # every other row untouched
    mask = torch.ones(cap, dtype=torch.bool)
    mask[pos] = False
    assert not kc[:, mask].any() and not vc[:, mask].any()
    # a full cache: position == capacity writes nothing
    p.fill_(cap)
    kc2 = torch.zeros_like(kc)
    assert D.lib().stark_decode_qk_norm_rope(_p(q), _p(k), _p(v), _p(qw), _p(kw), _p(kc2), _p(vc), _p(p), qh, kvh,
                                             cap, 1e6, 1e-6, _s()) == 0
    torch.cuda.synchronize()
    assert not kc2.any()


@pytest.mark.parametrize("qh,kvh", [(32, 8), (8, 8), (16, 8), (64, 8)])
@pytest.mark.parametrize("pos", [0, 127, 128, 300, 1023])
def test_attention(D, qh, kvh, pos):
    torch.manual_seed(qh + pos)
    cap = 1024
    q = torch.randn(qh * 128, device="cuda").to(torch.bfloat16)
    kc = torch.randn(kvh, cap, 128, device="cuda").to(torch.bfloat16)
    vc = torch.randn(kvh, cap, 128, device="cuda").to(torch.bfloat16)
    nch = D.lib().stark_decode_attn_chunks(cap)
    po = torch.empty(qh * nch * 128, device="cuda")
    pml = torch.empty(qh * nch * 2, device="cuda")
    out = torch.empty(qh * 128, dtype=torch.bfloat16, device="cuda")
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    assert D.lib().stark_decode_attention(_p(q), _p(kc), _p(vc), _p(po), _p(pml), _p(out), _p(p), qh, kvh, cap,
                                          _s()) == 0
    G = qh // kvh
    qf = q.float().view(kvh, G, 128)
    sc = torch.einsum("ghd,gpd->ghp", qf, kc[:, : pos + 1].float()) / np.sqrt(128.0)
    want = torch.einsum("ghp,gpd->ghd", torch.softmax(sc, -1), vc[:, : pos + 1].float()).reshape(-1)
    torch.testing.assert_close(out.float(), want, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("qh,kvh", [(32, 8), (8, 8), (16, 8), (64, 8)])
@pytest.mark.parametrize("pos", [0, 63, 64, 300, 1023, 1024])
def test_attention_fused_matches_two_kernels(D, qh, kvh, pos):
    """stark_decode_attention_fused (q/k norm + RoPE + KV write folded into the
    attention partials) against stark_decode_qk_norm_rope followed by
    stark_decode_attention on the same inputs; two calls in a row, the second
    at the next position; pos == capacity: a full cache takes no new row."""
    torch.manual_seed(qh * 7 + pos)
    cap = 1024
    nch = D.lib().stark_decode_attn_chunks(cap)
    qw = (1 + 0.1 * torch.randn(128, device="cuda")).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, device="cuda")).to(torch.bfloat16)
    kc = torch.randn(kvh, cap, 128, device="cuda").to(torch.bfloat16)
    vc = torch.randn(kvh, cap, 128, device="cuda").to(torch.bfloat16)
    kc2, vc2 = kc.clone(), vc.clone()
    for step in range(2):
        p_ = min(pos + step, cap)
        q = torch.randn(qh * 128, device="cuda").to(torch.bfloat16)
        k = torch.randn(kvh * 128, device="cuda").to(torch.bfloat16)
        v = torch.randn(kvh * 128, device="cuda").to(torch.bfloat16)
        p = torch.tensor([p_], dtype=torch.int32, device="cuda")
        po = torch.empty(qh * nch * 128, device="cuda")
        pml = torch.empty(qh * nch * 2, device="cuda")
        out = torch.empty(qh * 128, dtype=torch.bfloat16, device="cuda")
        assert D.lib().stark_decode_attention_fused(_p(q), _p(k), _p(v), _p(qw), _p(kw), _p(kc), _p(vc), _p(po),
                                                    _p(pml), _p(out), _p(p), qh, kvh, cap, 1e6, 1e-6, _s()) == 0
        q2 = q.clone()
        po2, pml2 = torch.empty_like(po), torch.empty_like(pml)
        out2 = torch.empty_like(out)
        assert D.lib().stark_decode_qk_norm_rope(_p(q2), _p(k), _p(v), _p(qw), _p(kw), _p(kc2), _p(vc2), _p(p), qh,
                                                 kvh, cap, 1e6, 1e-6, _s()) == 0
        assert D.lib().stark_decode_attention(_p(q2), _p(kc2), _p(vc2), _p(po2), _p(pml2), _p(out2), _p(p), qh, kvh,
                                              cap, _s()) == 0
        torch.cuda.synchronize()
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
        torch.testing.assert_close(out.float(), out2.float(), rtol=1e-2, atol=1e-2)


def test_attention_rejects_bad_heads(D):
    z = C.c_void_p(0)
    assert D.lib().stark_decode_attention(z, z, z, z, z, z, z, 32, 0, 64, _s()) == 1
    assert D.lib().stark_decode_attention(z, z, z, z, z, z, z, 30, 8, 64, _s()) == 1
    assert D.lib().stark_decode_attention(z, z, z, z, z, z, z, 96, 8, 64, _s()) == 1  # group 12


def test_silu_mul(D):
    torch.manual_seed(3)
    n = 12288 + 17
    g = (3 * torch.randn(n, device="cuda")).to(torch.bfloat16)
    u = torch.randn(n, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(g)
    assert D.lib().stark_decode_silu_mul(_p(g), _p(u), _p(out), n, _s()) == 0
    want = _bf(torch.nn.functional.silu(g.float())) * u.float()
    torch.testing.assert_close(out.float(), want, rtol=1e-2, atol=1e-3)


def test_argmax_and_embed(D):
    torch.manual_seed(4)
    n = 151936
    logits = torch.randn(n, device="cuda")
    logits[777] = 50.0
    logits[90000] = 50.0  # tie: the lower index wins
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos = torch.tensor([5], dtype=torch.int32, device="cuda")
    hist = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    assert D.lib().stark_decode_argmax(_p(logits), n, _p(tok), _p(pos), _p(hist), 8, _s()) == 0
    assert tok.item() == 777 and pos.item() == 6 and hist[5].item() == 777
    # a full history leaves the position where it is
    pos.fill_(8)
    assert D.lib().stark_decode_argmax(_p(logits), n, _p(tok), _p(pos), _p(hist), 8, _s()) == 0
    assert pos.item() == 8
    # ties inside one 16-byte chunk and across one thread's chunks, the last
    # element; then a count with a tail past the last whole chunk (1027 values)
    logits[777] = 0.0
    logits[90000] = 0.0
    for m, where in [(61.0, (4101, 4102)), (62.0, (8, 8 + 4096 * 4)), (63.0, (n - 1,))]:
        for w in where:
            logits[w] = m
        assert D.lib().stark_decode_argmax(_p(logits), n, _p(tok), _p(pos), _p(hist), 8, _s()) == 0
        assert tok.item() == where[0]
    odd = torch.randn(1027, device="cuda")
    odd[1026] = 99.0
    assert D.lib().stark_decode_argmax(_p(odd), 1027, _p(tok), _p(pos), _p(hist), 8, _s()) == 0
    assert tok.item() == 1026
    # all NaN: the token stays in range
    logits.fill_(float("nan"))
    assert D.lib().stark_decode_argmax(_p(logits), n, _p(tok), _p(pos), _p(hist), 8, _s()) == 0
    assert tok.item() == 0
    table = torch.randn(100, 512, device="cuda").to(torch.bfloat16)
    x = torch.empty(512, dtype=torch.bfloat16, device="cuda")
    tok.fill_(42)
    assert D.lib().stark_decode_embed(_p(table), _p(tok), _p(x), 512, 100, _s()) == 0
    assert torch.equal(x, table[42])
    tok.fill_(1000)  # out of range: clamped to the last row
    assert D.lib().stark_decode_embed(_p(table), _p(tok), _p(x), 512, 100, _s()) == 0
    assert torch.equal(x, table[99])


def _small(D, seed=0):
    cfg = D.Qwen3Config(hidden=512, layers=2, q_heads=8, kv_heads=2, head_dim=128, intermediate=1024, vocab=1000)
    return D.Qwen3Decoder(cfg, capacity=300, seed=seed)


def _deq(mat, group):
    n, k, bits = mat["n"], mat["k"], mat["bits"]
    c = mat["codes"]
    q = torch.stack([c & 15, c >> 4], -1).reshape(n, k) if bits == 4 else c
    s = mat["scales"].view(torch.bfloat16).float().t().repeat_interleave(group, 1)
    b = mat["biases"].view(torch.bfloat16).float().t().repeat_interleave(group, 1)
    return q.float() * s + b


def _reference_step(m, tok, pos):
    """Torch fp32 forward of one token over the dequantized weights, with the
    bf16 storage points of the kernels (residual, projections, norms, KV)."""
    cfg, g = m.cfg, m.cfg.group
    hd, G = cfg.head_dim, cfg.q_heads // cfg.kv_heads
    x = m.embed[tok].float()
    for L in m.layers:
        h = _rms(x, L["attn_norm"], cfg.eps)
        q = _bf(_deq(L["q"], g) @ h).view(cfg.q_heads, hd)
        k = _bf(_deq(L["k"], g) @ h).view(cfg.kv_heads, hd)
        v = _bf(_deq(L["v"], g) @ h).view(cfg.kv_heads, hd)
        q = _bf(_rope(_rms(q, L["q_norm"], cfg.eps), pos, cfg.rope_theta))
        k = _bf(_rope(_rms(k, L["k_norm"], cfg.eps), pos, cfg.rope_theta))
        K = L["kcache"][:, : pos + 1].float().clone()
        V = L["vcache"][:, : pos + 1].float().clone()
        K[:, pos], V[:, pos] = k, v
        sc = torch.einsum("ghd,gpd->ghp", q.view(cfg.kv_heads, G, hd), K) / np.sqrt(hd)
        att = _bf(torch.einsum("ghp,gpd->ghd", torch.softmax(sc, -1), V).reshape(-1))
        x = _bf(x + _deq(L["o"], g) @ att)
        h = _rms(x, L["mlp_norm"], cfg.eps)
        a = _bf(_bf(torch.nn.functional.silu(_bf(_deq(L["gate"], g) @ h))) * _bf(_deq(L["up"], g) @ h))
        x = _bf(x + _deq(L["down"], g) @ a)
    h = _rms(x, m.final_norm, cfg.eps)
    return _deq(m.lm_head, g) @ h


def test_decode_step_matches_torch(D):
    m = _small(D)
    m.fill_context(200)
    tok, pos = int(m.token.item()), int(m.pos.item())
    want = _reference_step(m, tok, pos)
    m.step()
    torch.cuda.synchronize()
    got = m.logits
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    assert err <= 2e-2 * scale, f"logits max err {err} vs scale {scale}"
    assert int(m.pos.item()) == pos + 1
    assert int(m.token.item()) == int(torch.argmax(got).item())
    assert int(m.history[pos].item()) == int(m.token.item())


def test_graph_replay_matches_eager(D):
    steps = 6
    eager = _small(D, seed=3)
    eager.fill_context(120)
    for _ in range(steps):
        eager.step()
    torch.cuda.synchronize()

    g = _small(D, seed=3)
    g.fill_context(120)
    g.step()  # builds schedules eagerly; the graph then runs the remaining steps
    torch.cuda.synchronize()
    graph = g.capture()
    # capture records without running: state is still one step in
    torch.cuda.synchronize()
    assert int(g.pos.item()) == 121
    for i in range(steps - 1):
        graph.replay()
        torch.cuda.synchronize()  # eager work between replays
        assert int(g.pos.item()) == 122 + i
    assert torch.equal(g.history[:120 + steps + 1], eager.history[:120 + steps + 1])
    assert torch.equal(g.logits, eager.logits)
    for La, Lb in zip(g.layers, eager.layers):
        assert torch.equal(La["kcache"][:, :120 + steps], Lb["kcache"][:, :120 + steps])
