"""GPU parity of GPT.forward (utils/model.py:193-210) on the population kernels.

The clean model runs as B members (one per batch row, each reading its own token sequence) with sigma = 0.
References:
* the bf16-mode oracle (the reference's autocast rounding points, fp32 head) for per-token losses,
  their reductions with ignore_index = -1, and the capped logits;
* the population path itself (`Population.loss` with sign 0 on each sequence alone), which must give the
  same per-sequence means: a wrong per-member token stride would feed every member sequence 0.

Tolerances: the north star's 1e-4 absolute bar on the mean loss at the reference's initialisation; per token,
twice the distance between the oracle and the same oracle accumulating in fp64 (its rounding floor; a single
token's loss moves by a few 1e-4 under such changes) plus 1e-4; <= 1e-2 relative on logits at trained-scale
weights (the bf16-activation bar)."""
import pytest
import torch
from torch.nn import functional as F

from noise_amd.model import make_model
from noise_amd.population import Population, clean_forward
from noise_amd.synthetic import trained_like, zipf_tokens
from oracle import model as om
from tests._util import log_case, rel_err

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _batch(B, T, seed):
    xs, ys = zip(*(zipf_tokens(T, seed=seed + b) for b in range(B)))
    return torch.stack(xs), torch.stack(ys)


def _zero_noise(params, rows=1):
    return {n: (torch.zeros(rows, t.shape[0]), torch.zeros(rows, t.shape[1])) if t.dim() == 2
            else torch.zeros(rows, t.shape[0]) for n, t in params.items()}


def _gpu_model(model):
    m = make_model('cpu', 0)
    m.load_state_dict(model.state_dict())
    return m.to(DEV)


def _oracle_logits(params, idx, fp64_accumulate=False):
    """Capped fp32-head logits [B, T, V] of the bf16-mode oracle, one sequence at a time (sigma = 0). With
    fp64_accumulate, every GEMM accumulates in fp64 (same bf16 rounding points): an equally valid rounding
    whose distance from the default measures how far the bf16 path's results move per token."""
    orig = om.lowrank

    def lowrank64(x, weight, a, b, s, mode='fp32'):
        if mode == 'fp32':
            return orig(x, weight, a, b, s, mode)
        u = om.bf((om.bf(x).double() @ om.bf(b).double().unsqueeze(-1)).float())
        dense = om.bf((om.bf(x).double() @ om.bf(weight).double().t()).float())
        return dense + s[:, None, None] * u * a[:, None, :]

    out = []
    if fp64_accumulate:
        om.lowrank = lowrank64
    try:
        for b in range(idx.shape[0]):
            _, h = om.population_loss(params, _zero_noise(params), torch.zeros(1), idx[b], idx[b], mode='bf16',
                                      head='fp32', return_hidden=True)
            z = (h[0] @ params['lm_head.weight'].t())[..., :om.VOCAB].float()
            out.append(om.SOFTCAP * torch.tanh(z / om.SOFTCAP))
    finally:
        om.lowrank = orig
    return torch.stack(out)


def _token_ce(logits, tgt):
    return F.cross_entropy(logits.view(-1, logits.shape[-1]), tgt.view(-1), ignore_index=-1, reduction='none')


def test_clean_forward_reductions_and_ignore_index_at_reference_init():
    model = make_model('cpu', 0)
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    B, T = 3, 256
    idx, tgt = _batch(B, T, seed=41)
    tgt[:, ::7] = -1  # ignored positions (ignore_index = -1, utils/model.py:207)
    log_case(f'clean_forward B={B} T={T} reference init')
    gm = _gpu_model(model)
    di, dt = idx.to(DEV), tgt.to(DEV)
    none = clean_forward(gm, di, dt, 'none').cpu()
    mean = clean_forward(gm, di, dt, 'mean').cpu()
    total = clean_forward(gm, di, dt, 'sum').cpu()
    via_module = gm(di, dt).cpu()  # GPT.forward dispatches to the same path
    ref = _token_ce(_oracle_logits(params, idx), tgt)
    # per-token rounding floor: how far one equally valid rounding (fp64 accumulation) moves each token's loss
    floor = float((_token_ce(_oracle_logits(params, idx, fp64_accumulate=True), tgt) - ref).abs().max())
    valid = tgt.view(-1) != -1
    assert none.shape == (B * T,) and mean.dim() == 0 and total.dim() == 0
    assert torch.all(none[~valid] == 0)
    assert (none - ref).abs().max() <= 2 * floor + 1e-4, (float((none - ref).abs().max()), floor)
    # the mean over the valid tokens: the north star's 1e-4 loss bar
    assert abs(float(mean) - float(ref[valid].mean())) < 1e-4, (float(mean), float(ref[valid].mean()))
    assert abs(float(total) - float(none.double().sum())) <= 1e-5 * abs(float(total))
    assert abs(float(mean) - float(none.double().sum() / valid.sum())) <= 1e-5 * abs(float(mean))
    assert torch.equal(via_module, mean)
    # every target ignored: the mean is NaN (as torch's), the sum 0
    allign = torch.full_like(dt, -1)
    assert torch.isnan(clean_forward(gm, di, allign, 'mean')).item()
    assert clean_forward(gm, di, allign, 'sum').item() == 0.0


def test_clean_forward_sequences_and_logits_at_trained_scale():
    torch.manual_seed(0)
    model = trained_like(make_model('cpu', 0))
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    B, T = 2, 256
    idx, tgt = _batch(B, T, seed=51)
    log_case(f'clean_forward B={B} T={T} trained-scale weights, logits')
    gm = _gpu_model(model)
    gp = dict(gm.named_parameters())
    di, dt = idx.to(DEV), tgt.to(DEV)
    none = clean_forward(gm, di, dt, 'none').cpu().view(B, T)
    # each sequence alone through the population path (sign 0): the same kernels, one shared sequence
    pop = Population(gm, chunk=1)
    zn = {n: tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV) for n, v in _zero_noise(params).items()}
    for b in range(B):
        alone = pop.loss(gp, zn, torch.zeros(1, device=DEV), di[b].contiguous(), dt[b].contiguous()).cpu()
        assert abs(float(alone[0]) - float(none[b].double().mean())) < 1e-5, (b, alone, none[b].mean())
    assert abs(float(none[0].mean()) - float(none[1].mean())) > 1e-3  # the sequences differ
    logits = clean_forward(gm, di).cpu()
    assert logits.shape == (B, T, 4096) and logits.dtype == torch.float32
    assert float(logits.abs().max()) <= 15.0
    # the logits and the losses come from the same capped values
    lse = torch.logsumexp(logits.double(), -1) - logits.double().gather(-1, tgt[..., None]).squeeze(-1)
    assert (lse - none.double()).abs().max() < 1e-4, float((lse - none.double()).abs().max())
    ref = _oracle_logits(params, idx)
    assert rel_err(logits, ref) < 1e-2, rel_err(logits, ref)


def _bf16_tables(params):
    """The reference's bf16 storage of the token and value embeddings on a GPU (utils/model.py:171-175)."""
    for k in ['transformer.wte.weight'] + [k for k in params if k.startswith('value_embeds.')]:
        params[k] = params[k].bfloat16().float()
    return params


def test_evaluate_score_matches_oracle_with_ragged_batches():
    """utils/eval.py's evaluate: bf16 embedding storage, fp64 sums over ragged batches. The default rounding is
    utils/eval.py's autocast (the autocast oracle); rounding='population' keeps the population path's."""
    from noise_amd.eval import evaluate
    model = make_model('cpu', 0)
    sd = model.state_dict()
    n, T = 4, 256
    rows = torch.stack([torch.cat([i, t[-1:]]) for i, t in (zipf_tokens(T, seed=61 + r) for r in range(n))])
    log_case(f'evaluate rows={n} T={T} batch 3')
    got = evaluate(sd, rows=rows, batch_size=3)
    params = _bf16_tables({k: v.detach().clone() for k, v in model.named_parameters()})
    ref = om.autocast_forward(params, rows[:, :-1], rows[:, 1:], 'none').double().mean()
    assert abs(got - float(ref)) < 1e-4, (got, float(ref))
    got_pop = evaluate(sd, rows=rows, batch_size=3, rounding='population')
    ref_pop = torch.cat([om.population_loss(params, _zero_noise(params), torch.zeros(1), r[:-1], r[1:], mode='bf16',
                                            head='bf16') for r in rows]).double().mean()
    assert abs(got_pop - float(ref_pop)) < 1e-4, (got_pop, float(ref_pop))


@pytest.mark.parametrize('trained', [False, True])
def test_autocast_forward_matches_the_autocast_oracle(trained):
    """GPT.forward at utils/eval.py's rounding (bf16 autocast, bf16 tables) against oracle.model.autocast_forward.
    Per token and for the mean: within twice the oracle's own floor (the distance to the same oracle accumulating
    its GEMMs in fp64, an equally valid rounding) plus 1e-4; at the reference init that is the 1e-4 bar on the
    mean. Logits within 1e-2 relative. Under torch.autocast('cuda', bfloat16) GPT.forward takes this path."""
    from noise_amd.population import autocast_forward
    torch.manual_seed(0)
    model = trained_like(make_model('cpu', 0)) if trained else make_model('cpu', 0)
    params = _bf16_tables({n: p.detach().clone() for n, p in model.named_parameters()})
    B, T = 2, 256
    idx, tgt = _batch(B, T, seed=71)
    log_case(f'autocast_forward B={B} T={T} trained={trained}')
    gm = _gpu_model(model)
    di, dt = idx.to(DEV), tgt.to(DEV)
    none = autocast_forward(gm, di, dt, 'none').cpu()
    mean = autocast_forward(gm, di, dt, 'mean').cpu()
    with torch.autocast('cuda', dtype=torch.bfloat16):
        via_module = gm(di, dt).cpu()
    assert torch.equal(via_module, mean)
    ref = om.autocast_forward(params, idx, tgt, 'none')
    ref64 = om.autocast_forward(params, idx, tgt, 'none', accumulate=torch.float64)
    floor_tok = float((ref64 - ref).abs().max())
    floor_mean = abs(float(ref64.double().mean() - ref.double().mean()))
    err_tok = float((none - ref).abs().max())
    err_mean = abs(float(mean) - float(ref.double().mean()))
    assert err_tok <= 2 * floor_tok + 1e-4, (err_tok, floor_tok)
    assert err_mean <= 2 * floor_mean + 1e-4, (err_mean, floor_mean)
    if not trained:
        assert err_mean < 1e-4, err_mean
    # the logits are bf16 values (the head's autocast output): within 1e-2 relative, or twice the oracle's own floor
    # where one-ulp flips upstream move more than that (reference init: 0.4e-2 of bf16 rounding per logit alone)
    logits = autocast_forward(gm, di).cpu()
    assert logits.shape == (B, T, 4096) and logits.dtype == torch.float32
    ref_l = om.autocast_forward(params, idx)
    floor_l = rel_err(om.autocast_forward(params, idx, accumulate=torch.float64), ref_l)
    assert rel_err(logits, ref_l) <= max(1e-2, 2 * floor_l), (rel_err(logits, ref_l), floor_l)
