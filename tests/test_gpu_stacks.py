"""BASELINE configs 3 and 4 on the GPU: the path's kernels at the stacks' full shapes, and the
random-init stacks end to end (xlstm_hip.stack).

* config 3 (xLSTM-7B shapes): the mLSTM layer's prefill at B1 NH8 S2048 DQK256 DV512 bf16 on the
  q, k, v and gates a random-init block projects from a random input, against the oracle on the
  whole batch (h and the last C, n, m); one decode step from those states (B1 NH8);
* config 4: the mLSTM heads at B8 NH8 DQK128 DV256 S4096 and the sLSTM layer's time loop at
  B8 S4096 NH4 H512 (z and gates from a random-init sLSTM block's projection cell), each against
  the oracle at full size;
* both stacks at full size (config 3: 32 blocks, d 4096, prompt 2048; config 4: 24 blocks with 3
  sLSTM blocks, d 2048, B8, prompt 4096): finite logits, greedy decoding deterministic from run to
  run, and the HIP-graph decode step (replayed once per token, with eager work and host syncs
  between replays) giving the eager decoder's tokens.
"""

import pytest
import torch

from helpers import assert_parity, dev, print_margins
from oracle import mlstm as om
from oracle import slstm as osl

pytestmark = pytest.mark.gpu


def _block_inputs(block, B, S, d, seed):
    # a stream of its own: drawn with the weights' seed, x would correlate with the weights
    g = torch.Generator(device=dev()).manual_seed(10_000 + seed)
    x = torch.randn(B, S, d, generator=g, device=dev()).to(torch.bfloat16)
    return block.norm_mlstm(x) if hasattr(block, "norm_mlstm") else block.norm_slstm(x)


def _mlstm_qkvif(cfg, B, S, seed):
    from xlstm_hip.stack import _mLSTMBlock
    blk = _mLSTMBlock(cfg).to(torch.bfloat16).to(dev())
    torch.manual_seed(seed)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if "norm" in name:
                p.fill_(1.0)
            elif name.endswith("fgate_proj.bias"):
                p.fill_(3.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                p.normal_(0.0, cfg.init_std)
        xn = _block_inputs(blk, B, S, cfg.d_model, seed)
        q, k, v, i, f = blk.proj(xn)
    return blk, tuple(t.contiguous() for t in (q, k, v, i, f))


def _check_chunkwise(x, name):
    import xlstm_hip
    q, k, v, i, f = x
    h, (C, n, m) = xlstm_hip.mlstm_chunkwise(q, k, v, i, f, return_last_states=True)
    hr, (Cr, nr, mr) = om.mlstm_chunkwise(*(t.float().cpu() for t in x), return_last_states=True)
    for got, want, nm in ((h, hr, "h"), (C, Cr, "C"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got.cpu(), want, torch.bfloat16, f"{name} {nm}")
    return (C, n, m), (Cr, nr, mr)


def test_cfg3_mlstm_layer_prefill_and_decode(gpu_case):
    import xlstm_hip
    from xlstm_hip.stack import CFG3_STACK as cfg
    blk, x = _mlstm_qkvif(cfg, 1, 2048, seed=31)
    q, k, v, i, f = x
    assert q.shape == (1, 8, 2048, 256) and v.shape == (1, 8, 2048, 512) and i.shape == (1, 8, 2048)
    assert float(torch.cat([i, f]).float().abs().max()) <= 15.0  # soft-capped at 15
    assert 2.5 < float(f.float().mean()) < 3.5  # the forget-gate bias
    (C, n, m), (Cr, nr, mr) = _check_chunkwise(x, "cfg3 prefill")
    # one decode step from the prefill's states (the in-place serving step)
    with torch.no_grad():
        xn = _block_inputs(blk, 1, 1, cfg.d_model, seed=32)
        q1, k1, v1, i1, f1 = blk.proj(xn)
    C2 = C.clone()
    h, (_, n2, m2) = xlstm_hip.mlstm_recurrent_step_(q1[:, :, 0], k1[:, :, 0], v1[:, :, 0], i1, f1, C2, n, m)
    hr, (C2r, n2r, m2r) = om.mlstm_recurrent_step(q1[:, :, 0].cpu(), k1[:, :, 0].cpu(), v1[:, :, 0].cpu(),
                                                  i1.float().cpu(), f1.float().cpu(), C.cpu(), n.cpu(), m.cpu())
    # h with a bf16 q: the reference's three bf16 roundings of it (q C', q n', the quotient), any of
    # which a 1-ulp difference of the gate exponentials can flip (tests/test_oracle_bf16_sensitivity.py)
    print_margins(h.cpu(), hr, "cfg3 decode h")
    for got, want, nm in ((h, hr, "h"), (C2, C2r, "C"), (n2, n2r, "n"), (m2, m2r, "m")):
        assert_parity(got.cpu(), want, torch.bfloat16, f"cfg3 decode {nm}", roundings=3 if nm == "h" else 1)


def test_cfg4_mlstm_heads_full(gpu_case):
    from xlstm_hip.stack import CFG4_STACK as cfg
    _, x = _mlstm_qkvif(cfg, 8, 4096, seed=41)
    assert x[0].shape == (8, 8, 4096, 128) and x[2].shape == (8, 8, 4096, 256)
    _check_chunkwise(x, "cfg4 mLSTM heads")


def test_cfg4_slstm_layer_full(gpu_case):
    import xlstm_hip
    from xlstm_hip.stack import CFG4_STACK as cfg, _sLSTMBlock
    blk = _sLSTMBlock(cfg).to(torch.bfloat16).to(dev())
    torch.manual_seed(42)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if "norm" in name:
                p.fill_(1.0)
            elif name.endswith("fgate_proj.bias"):
                p.fill_(3.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                p.normal_(0.0, 0.02)
        xn = _block_inputs(blk, 8, 4096, cfg.d_model, seed=43)
        z, i, f, o, _ = blk.proj(xn)
    z, i, f, o = (t.contiguous() for t in (z, i, f, o))
    assert z.shape == (8, 4096, 4, 512) and i.shape == (8, 4096, 4)
    h, (c, n, m) = xlstm_hip.slstm_sequence(z, i, f, o)
    hr, (cr, nr, mr) = osl.slstm_sequence(*(t.float().cpu() for t in (z, i, f, o)))
    assert h.dtype == torch.bfloat16
    for got, want, nm in ((h, hr, "h"), (c, cr, "c"), (n, nr, "n"), (m, mr, "m")):
        assert_parity(got.cpu(), want, torch.bfloat16, f"cfg4 sLSTM {nm}")


@pytest.mark.parametrize("which", ["cfg3", "cfg4"])
def test_stack_end_to_end(gpu_case, which):
    from xlstm_hip.stack import CFG3_STACK, CFG4_STACK, DecodeGraph, xLSTMStack
    cfg, B, S = (CFG3_STACK, 1, 2048) if which == "cfg3" else (CFG4_STACK, 8, 4096)
    steps = 6
    model = xLSTMStack.random(cfg, dev(), seed=7)
    g = torch.Generator(device=dev()).manual_seed(8)
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=g, device=dev())
    logits, states = model.prefill(prompt)
    assert logits.shape == (B, cfg.vocab) and bool(torch.isfinite(logits.float()).all())
    assert float(logits.float().abs().max()) <= cfg.logit_soft_cap
    # eager greedy decode, twice from scratch: identical tokens
    runs = []
    for _ in range(2):
        logits, states = model.prefill(prompt)
        tok, out = logits.argmax(-1), []
        for _ in range(steps):
            out.append(tok)
            lg = model.decode_step(tok, states)
            assert bool(torch.isfinite(lg.float()).all())
            tok = lg.argmax(-1)
        runs.append(torch.stack(out, 1))
    assert torch.equal(runs[0], runs[1])
    # graph decode: one replay per token, eager work and host syncs between replays
    logits, states = model.prefill(prompt)
    dg = DecodeGraph(model, states, logits.argmax(-1))
    toks = []
    for t in range(steps):
        toks.append(dg.step())
        torch.cuda.synchronize()
        _ = torch.ones(16, device=dev()).sum().item()
        assert torch.equal(toks[-1], runs[0][:, t]), f"{which}: graph decode token {t} differs from eager"


@pytest.mark.parametrize("S", [200, 256])
def test_stack_prefill_decode_handoff(gpu_case, S):
    """prefill(tokens[:S]) followed by decode_step(tokens[S]) gives the logits of
    prefill(tokens[:S + 1]), on a reduced stack of two mLSTM and two sLSTM blocks (cfg4's head
    shapes): every state the prefill hands to decode -- each mLSTM block's C, n, m, each sLSTM
    block's c, n, m and its conv window, the capped gates of the step -- is the one the longer
    prefill carries through token S.  The two sides run different kernels (chunkwise and sLSTM
    sequence kernels against the step kernels) in bf16, so they agree to bf16 roundings amplified
    through four blocks (measured 2-4 % of the largest logit; bar 5 %), not bit for bit; dropping
    the context moves the logits by more than the largest logit (checked, so the bar can tell)."""
    from xlstm_hip.stack import StackConfig, xLSTMStack
    cfg = StackConfig("handoff", d_model=2048, num_blocks=4, mlstm_heads=8, slstm_every=2, vocab=4096,
                      init_std=0.05)
    model = xLSTMStack.random(cfg, dev(), seed=17)
    g = torch.Generator(device=dev()).manual_seed(18)
    tokens = torch.randint(0, cfg.vocab, (2, S + 1), generator=g, device=dev())
    want, _ = model.prefill(tokens)
    _, states = model.prefill(tokens[:, :S])
    got = model.decode_step(tokens[:, S], states)
    diff = float((got.float() - want.float()).abs().max())
    scale = float(want.float().abs().max())
    # how far the logits move without the context (token S alone, every state from zero): what
    # a hand-off that lost the states would give; the bar must sit well below it
    alone, _ = model.prefill(tokens[:, S:S + 1])
    ctx = float((alone.float() - want.float()).abs().max())
    print(f"[handoff] S={S}: max |decode - prefill| {diff:.3e}, without the context {ctx:.3e} "
          f"(max |logit| {scale:.3e})")
    assert bool(torch.isfinite(got.float()).all())
    bar = 0.05 * scale
    assert ctx >= 4 * bar, f"the context moves the logits by only {ctx:.3e}: the check cannot tell"
    assert diff <= bar, f"prefill -> decode hand-off: logits differ by {diff:.3e}"
