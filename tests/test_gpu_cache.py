"""GPU checks of the recurrent cache through the layer adapter: token-by-token
decoding equals the dense call (the reference's
test_modeling_solvedelta.py:263-301 gate, rtol 1e-2 / atol 2e-2, at the layer),
split prefill + continuation equals one call (:235-260), prefill + decode
against the FP64 mixer oracle, and the cached state
has the wire format (fp32 (C, S), conv [B, 2Hr + HV, 3])."""
import pytest
import torch

from gpu_common import rel

pytestmark = pytest.mark.gpu


def _adapter(hidden=128, H=1, r=128, seed=6):
    from solvedelta_amd import SolveDeltaMixerConfig
    from solvedelta_amd.cache import SolveDeltaCacheAdapter
    torch.manual_seed(seed)
    cfg = SolveDeltaMixerConfig(hidden_size=hidden, num_heads=H, head_k_dim=r, head_v_dim=r)
    return SolveDeltaCacheAdapter(cfg, layer_idx=0).cuda().to(torch.bfloat16).eval()


def test_single_token_cache_matches_dense():
    from solvedelta_amd.cache import RecurrentCache
    ad = _adapter()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 16, 128, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        dense, _, _ = ad(x, use_cache=False)
        cache = RecurrentCache()
        pieces = []
        for t in range(16):
            y, _, cache = ad(x[:, t:t + 1], past_key_values=cache, use_cache=True)
            pieces.append(y)
    rec = torch.cat(pieces, 1)
    print(f"[cache T=1 x16] rel {rel(rec.float(), dense.float()):.2e}", flush=True)
    torch.testing.assert_close(rec.float(), dense.float(), rtol=1e-2, atol=2e-2)
    assert cache.get_seq_length() == 16
    C, S = cache[0]["recurrent_state"]
    assert C.dtype == torch.float32 and S.dtype == torch.float32
    assert C.shape == (1, 1, 128, 128) and S.shape == (1, 1, 128, 128)
    assert cache[0]["conv_state"].shape == (1, 2 * 128 + 128, 3)


def test_split_prefill_matches_whole():
    from solvedelta_amd.cache import RecurrentCache
    ad = _adapter(hidden=64, H=2, r=32, seed=5)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 9, 64, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        whole, _, _ = ad(x)
        cache = RecurrentCache()
        left, _, cache = ad(x[:, :4], past_key_values=cache, use_cache=True)
        right, _, cache = ad(x[:, 4:], past_key_values=cache, use_cache=True)
    e = rel(right.float(), whole[:, 4:].float())
    print(f"[cache split 4+5] rel {e:.2e}", flush=True)
    assert e < 1e-2
    assert cache.get_seq_length() == 9


def test_packed_cu_seqlens_equal_separate_sequences():
    ad = _adapter(hidden=64, H=2, r=32, seed=7)
    g = torch.Generator().manual_seed(3)
    a = torch.randn(1, 5, 64, generator=g).to(torch.bfloat16).cuda()
    b = torch.randn(1, 7, 64, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        packed, _, _ = ad(torch.cat((a, b), 1),
                          cu_seqlens=torch.tensor([0, 5, 12], dtype=torch.int32, device="cuda"))
        ya, _, _ = ad(a)
        yb, _, _ = ad(b)
    e = rel(packed.float(), torch.cat((ya, yb), 1).float())
    print(f"[cache packed] rel {e:.2e}", flush=True)
    assert e < 1e-2


def test_cache_prefill_then_decode_matches_mixer_oracle():
    """Prefill 9 tokens, then 16 single-token steps through the cache, each
    carrying (C, S, conv) in the wire format; outputs and the final cached state
    against the FP64 mixer oracle run densely over all 25 tokens."""
    from oracle.mixer_oracle import mixer_oracle
    from solvedelta_amd.cache import RecurrentCache
    ad = _adapter(hidden=128, H=2, r=64, seed=12)
    with torch.no_grad():
        ad.mixer.output_norm.weight.uniform_(0.5, 1.5)
    g = torch.Generator().manual_seed(13)
    x = torch.randn(2, 25, 128, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        cache = RecurrentCache()
        y0, _, cache = ad(x[:, :9], past_key_values=cache, use_cache=True)
        pieces = [y0]
        for t in range(9, 25):
            y, _, cache = ad(x[:, t:t + 1], past_key_values=cache, use_cache=True)
            pieces.append(y)
    rec = torch.cat(pieces, 1)
    params = {k: v.detach().double().cpu() for k, v in ad.mixer.named_parameters()}
    yo, (Co, So), conv_o = mixer_oracle(params, x.double().cpu(), heads=2, rk=64, rv=64)
    C, S = cache[0]["recurrent_state"]
    conv = cache[0]["conv_state"]
    ey, eC, eS, ec = rel(rec.float(), yo), rel(C, Co), rel(S, So), rel(conv.float(), conv_o)
    print(f"[cache vs oracle] rel y {ey:.2e} C {eC:.2e} S {eS:.2e} conv {ec:.2e}", flush=True)
    torch.testing.assert_close(rec.float().cpu(), yo.float(), rtol=1e-2, atol=2e-2)
    assert ey < 3e-2 and eC < 3e-2 and eS < 3e-2 and ec < 1e-2
    assert cache.get_seq_length() == 25
