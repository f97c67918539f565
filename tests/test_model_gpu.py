"""End-to-end RWKV-7 decode step (vkwr.model_executor) against the
float32 composition oracle (oracle/model_ref.py).

Bar (north_star): end-to-end logits within max-abs 5e-2 of the float32 model;
slots outside the batch bitwise unchanged.  Both GEMM paths of the engine are
checked: the fragment-layout decode GEMM (default) and the row-major GEMM.
With the frag path the low-rank activations are rounded once (tanh / sigmoid
of the fp32 accumulator) where the oracle's round_fp16 mode rounds twice; the
tiny-model 1e-2 bound covers that one-ulp difference.  The WKV op itself is bit-exact on
identical inputs (tests/test_wkv_gpu.py); end to end its inputs differ from the
oracle's by fp16 rounding flips of the intermediates (GEMM accumulation order),
so the updated states are checked to the drift this produces: 1e-3 for the
2-layer model, 2.5e-2 after 24 layers of the 1.5B shape (measured on MI355X:
1.8e-3 at layer 0 rising to 1.0e-2 at layer 24, logits max-abs 2.4e-2 on
logits of magnitude up to 5).
"""
import pytest
import torch

from oracle import model_ref

pytestmark = pytest.mark.gpu

LOGIT_TOL = 5e-2
STATE_TOL = 1e-3


def _setup(gpu, preset, B, P, seed=0, frag=True):
    from vkwr_amd import capi
    from vkwr.model_executor import RWKV7Config, RWKV7Model, RWKV7State, DecodeEngine
    cfg = RWKV7Config.preset(preset)
    model = RWKV7Model(cfg, gpu, seed=seed)
    layout = capi.WKV_STATE_ILV if frag else capi.WKV_STATE_STD
    state = RWKV7State(cfg, P, gpu, std=0.1, seed=seed + 1, layout=layout)
    eng = DecodeEngine(model, B, frag=frag)
    g = torch.Generator().manual_seed(seed)
    slots = torch.randperm(P, generator=g)[:B].to(torch.int32).to(gpu)
    return cfg, model, state, eng, slots, g


@pytest.mark.parametrize("frag", [True, False], ids=["frag_gemm", "rowmajor_gemm"])
def test_tiny_model_matches_cpu_oracle_over_steps(gpu, frag):
    cfg, model, state, eng, slots, g = _setup(gpu, "tiny", B=4, P=9, frag=frag)
    wkv = state.wkv_standard().cpu()
    wkv0 = wkv.clone()
    att, ffn = state.att_shift.cpu().clone(), state.ffn_shift.cpu().clone()
    wkv_r, att_r, ffn_r = wkv.clone(), att.clone(), ffn.clone()
    for step in range(3):
        tokens = torch.randint(0, cfg.vocab, (4,), generator=g, dtype=torch.int32)
        logits = eng.step(state, tokens.to(gpu), slots).float().cpu()
        ref = model_ref.decode_step(model, wkv, att, ffn, tokens, slots.cpu(), round_fp16=True)
        ref32 = model_ref.decode_step(model, wkv_r, att_r, ffn_r, tokens, slots.cpu(), round_fp16=False)
        assert (logits - ref).abs().max() <= 1e-2, (step, float((logits - ref).abs().max()))
        assert (logits - ref32).abs().max() <= LOGIT_TOL, (step, float((logits - ref32).abs().max()))
        assert (state.wkv_standard().cpu() - wkv).abs().max() <= STATE_TOL
    others = [s for s in range(9) if s not in slots.cpu().tolist()]
    assert torch.equal(state.wkv_standard().cpu()[:, others], wkv0[:, others])


@pytest.mark.parametrize("frag", [True, False], ids=["frag_gemm", "rowmajor_gemm"])
def test_1p5b_decode_step_bs128_logits(gpu, frag):
    """BASELINE config 3 at full shape: L=24, C=2048, bs=128, one decode step, logits
    and states against the float32 composition evaluated with torch on the GPU."""
    cfg, model, state, eng, slots, g = _setup(gpu, "1.5b", B=128, P=160, frag=frag)
    tokens = torch.randint(0, cfg.vocab, (128,), generator=g, dtype=torch.int32).to(gpu)
    wkv = state.wkv_standard()
    wkv0 = wkv.clone()
    att, ffn = state.att_shift.clone(), state.ffn_shift.clone()
    logits = eng.step(state, tokens, slots).float()
    torch.cuda.synchronize()
    with torch.no_grad():
        ref = model_ref.decode_step(model, wkv, att, ffn, tokens, slots, round_fp16=False)
    err = (logits - ref).abs().max().item()
    assert err <= LOGIT_TOL, err
    sl = slots.long()
    got = state.wkv_standard()
    assert (got[:, sl] - wkv[:, sl]).abs().max().item() <= 2.5e-2
    others = torch.ones(160, dtype=torch.bool, device=gpu)
    others[sl] = False
    assert torch.equal(got[:, others], wkv0[:, others])  # untouched


@pytest.mark.parametrize("frag", [True, False], ids=["frag_gemm", "rowmajor_gemm"])
def test_decode_step_is_deterministic_and_graph_capturable(gpu, frag):
    cfg, model, state, eng, slots, g = _setup(gpu, "tiny", B=8, P=8, frag=frag)
    tokens = torch.randint(0, cfg.vocab, (8,), generator=g, dtype=torch.int32).to(gpu)
    s0 = [state.wkv.clone(), state.att_shift.clone(), state.ffn_shift.clone()]
    eager = eng.step(state, tokens, slots).clone()
    s1 = [state.wkv.clone(), state.att_shift.clone(), state.ffn_shift.clone()]
    # reset and replay through a captured graph, several times, eager work in between
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    for t, v in zip((state.wkv, state.att_shift, state.ffn_shift), s0):
        t.copy_(v)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = eng.step(state, tokens, slots)
    torch.cuda.synchronize()
    for _ in range(3):
        for t, v in zip((state.wkv, state.att_shift, state.ffn_shift), s0):
            t.copy_(v)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        for t, v in zip((state.wkv, state.att_shift, state.ffn_shift), s1):
            assert torch.equal(t, v)
