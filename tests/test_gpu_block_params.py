"""GPU parity of the transformer block's one-launch parameter gradients.

With LayerNorm norms and a sequence length that is a multiple of the
LayerNorm backward's 16-row blocks, the block's backward
(transformer.go:1220-1279) keeps the norms' block partials: the gamma / beta
sums, and the column sums of dx, which are the per-sample token sums that the
Q10 weight gradients of wOut and ff2 need.  The fused attention backward forms
the token sums of gQ, gK and gV.  Every parameter gradient of the block (six
Linear layers, two LayerNorms) then comes from one `tb_params` launch, and a
CLSPooling above the block (transformer.go:1679-1725) costs no launch: the
last norm's forward writes the pooled rows and its backward reads the pooled
gradient.  A PositionalEncoding over an Embedding has its gradient summed by
the Embedding's gradient launch, and the token sums of ff1's dz ride on the
norm-1 backward's launch.

Each case runs two training steps against the oracle (gpuutil.compare_step,
every tensor to 1e-4) from a random block, and checks from the per-launch
timing records which path ran: RMSNorm norms, or a sequence length that lets
a 16-row block span two samples, keep the per-layer token sums and Q10
launches.
"""
import pytest

from gpuutil import compare_step, log, random_block
from test_gpu_tail import _kernel_names

pytestmark = pytest.mark.gpu

FUSED = {"tb_params", "ln_bwd", "attn_bwd"}  # and the Embedding's gradient launch (embed_grad*)
UNFUSED = {"tok_dw", "cls_bwd", "cls_fwd", "token_sum"}


def cases():
    """name -> (gpt() arguments, workers, fused)"""
    return {
        # the fused path: causal, W = 1 and 3 (samples split over workers)
        "ln_t32": (dict(B=6, T=32, vocab=41, dim=32, heads=2, ff=48), 1, True),
        "ln_t48_w3": (dict(B=7, T=48, vocab=29, dim=64, heads=4, ff=40), 3, True),
        # non-causal, GELU feed-forward
        "ln_gelu": (dict(B=5, T=16, vocab=23, dim=32, heads=4, ff=24, causal=False, act="gelu"), 1, True),
        # RoPE rotates gQ, gK after the attention backward: their token sums
        # by launch, the rest fused
        "ln_rope": (dict(B=4, T=32, vocab=19, dim=32, heads=2, ff=32, rope=True), 2, True),
        # SwiGLU feed-forward (its ff1 gradient by GEMM), LayerNorm norms
        "ln_swiglu": (dict(B=4, T=16, vocab=31, dim=32, heads=2, ff=40, act="swiglu"), 1, True),
        # 144 tokens: batched-GEMM attention, fused parameter launch
        "ln_t144": (dict(B=3, T=144, vocab=17, dim=64, heads=2, ff=24), 1, True),
        # not fused: RMSNorm norms, and 20 tokens (16-row blocks span samples)
        "rms": (dict(B=5, T=32, vocab=37, dim=32, heads=4, ff=48, norm="rms"), 1, False),
        "ln_t20": (dict(B=6, T=20, vocab=41, dim=32, heads=2, ff=48), 2, False),
    }


@pytest.mark.parametrize("name", sorted(cases()))
def test_block_param_gradients(gn, oracle, dev, name):
    from goneuron_amd import configs
    kw, workers, fused = cases()[name]
    cfg = configs.gpt(**kw)
    compare_step(gn, oracle, cfg, steps=2, workers=workers, perturb=random_block(cfg))
    model = configs.build(cfg, workers=workers)
    x, y = configs.inputs(cfg)
    names = _kernel_names(dev, model, x, y)
    model.Close()
    log(f"{name}: {sorted(names)}")
    if fused:
        absent = set(UNFUSED)
        if kw.get("rope") or kw["T"] > 128:
            # gQ, gK rotated after the attention backward, or the batched-GEMM
            # attention: the token sums of gQ, gK, gV by launch
            absent.discard("token_sum")
        assert FUSED <= names and not (absent & names), sorted(names)
        assert any(n.startswith("embed_grad") for n in names), sorted(names)
    else:
        assert "tok_dw" in names and "tb_params" not in names, sorted(names)
