"""Host-side checks of the fused MLP's per-step weight-form cache (no GPU).

backward looks up the transposed bf16 LoRA forms by the ids of the five tensors _MLP saves (S, bg, bu, ad, bd).
When a saved-tensor hook hands backward fresh objects, an object that died after one layer's backward could
leave its address to the next layer's tensor; a lookup by id alone would then return the first layer's forms.
The cache entries hold their key tensors and a hit must be the very objects passed in, so that cannot happen.
These tests build forms for a run of short-lived key sets, as a cloning unpack hook does layer by layer, and
check every lookup against the tensors it was given; one of them makes every equal-shaped tensor share an id
(the worst case of address reuse).  The native prep call is replaced by the same casts and transposes in
torch."""
import gc

import torch

import _native
import fused_linear
import fused_mlp


def _torch_prep(Ag, Au, Bg, Bu, Ad, Bd, out):
    bf = torch.bfloat16
    S = torch.cat([Ag, Au]).to(bf)
    forms = dict(S=S, ST=S.t(), bg=Bg.to(bf), bu=Bu.to(bf), bgT=Bg.t().to(bf), buT=Bu.t().to(bf), ad=Ad.to(bf),
                 adT=Ad.t().to(bf), bd=Bd.to(bf), bdT=Bd.t().to(bf))
    for k, v in forms.items():
        out[k].copy_(v)


def _keys(seed, R=4, K=8, N=12):
    g = torch.Generator().manual_seed(seed)
    r = lambda *sh: torch.randn(*sh, generator=g).to(torch.bfloat16)  # noqa: E731
    return r(2 * R, K), r(N, R), r(N, R), r(R, N), r(K, R)


def _check_run(n=40):
    fused_linear.new_step()
    for seed in range(n):
        S, bg, bu, ad, bd = _keys(seed)
        lw = fused_mlp._forms_of_saved(S, bg, bu, ad, bd, torch.bfloat16)
        assert torch.equal(lw.bgT, bg.t()) and torch.equal(lw.adT, ad.t()) and torch.equal(lw.bdT, bd.t())
        assert torch.equal(lw.ST, S.t()) and torch.equal(lw.buT, bu.t())
        del S, bg, bu, ad, bd, lw
        gc.collect()
    fused_linear.new_step()


def test_forms_follow_short_lived_keys(monkeypatch):
    monkeypatch.setattr(_native, "lora_prep", _torch_prep)
    _check_run()


def test_forms_follow_keys_whose_ids_collide(monkeypatch):
    monkeypatch.setattr(_native, "lora_prep", _torch_prep)
    monkeypatch.setattr(fused_mlp, "id", lambda t: hash(tuple(t.shape)), raising=False)
    _check_run(8)


def test_forward_entry_is_found_by_the_same_objects(monkeypatch):
    monkeypatch.setattr(_native, "lora_prep", _torch_prep)
    fused_linear.new_step()
    S, bg, bu, ad, bd = _keys(7)
    first = fused_mlp._forms_of_saved(S, bg, bu, ad, bd, torch.bfloat16)
    assert fused_mlp._forms_of_saved(S, bg, bu, ad, bd, torch.bfloat16) is first
    # equal values in other objects: a separate entry, never the first one's
    S2, bg2, bu2, ad2, bd2 = (t.clone() for t in (S, bg, bu, ad, bd))
    other = fused_mlp._forms_of_saved(S2, bg2, bu2, ad2, bd2, torch.bfloat16)
    assert other is not first and other.keep[0] is S2
    fused_linear.new_step()
