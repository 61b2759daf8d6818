"""The oracle and the host-side init against golden vectors written by the reference itself
(tests/golden/make_golden.py imported /root/reference on the CPU). CPU only."""
import hashlib

import pytest
import torch

from noise_amd.model import make_model, window_sizes, GPTConfig
from noise_amd.synthetic import antithetic_signs, population_noise, trained_like, zipf_tokens
from oracle import eggroll as oe
from oracle import model as om

torch.set_num_threads(8)


def sha(t):
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def noise_sha(noise):
    h = hashlib.sha256()
    for name, n in noise.items():
        for t in (n if isinstance(n, tuple) else (n,)):
            h.update(name.encode())
            h.update(t.contiguous().numpy().tobytes())
    return h.hexdigest()


@pytest.fixture(scope='module')
def ref_inputs(golden):
    model = make_model('cpu', 0)
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    shapes = {n: tuple(p.shape) for n, p in params.items()}
    idx, targets = zipf_tokens(golden['T'])
    noise = population_noise(shapes, golden['pairs'])
    sign = antithetic_signs(2 * golden['pairs'], golden['sigma'])
    return model, params, shapes, idx, targets, noise, sign


def test_make_model_is_bit_exact(golden, ref_inputs):
    model = ref_inputs[0]
    sd = model.state_dict()
    assert set(sd) == set(golden['weights_sha256'])  # strict state-dict key set
    for name, digest in golden['weights_sha256'].items():
        assert sha(sd[name]) == digest, name


def test_rotary_and_windows(golden, ref_inputs):
    model = ref_inputs[0]
    assert sha(model.cos) == golden['rotary_sha256']['cos']
    assert sha(model.sin) == golden['rotary_sha256']['sin']
    cos, sin = om.rotary_tables()
    assert sha(cos[None, :, None, :]) == golden['rotary_sha256']['cos']
    assert sha(sin[None, :, None, :]) == golden['rotary_sha256']['sin']
    assert window_sizes(GPTConfig()) == golden['window_sizes'] == om.window_sizes()


def test_synthetic_inputs_unchanged(golden, ref_inputs):
    _, _, _, idx, targets, noise, _ = ref_inputs
    assert sha(idx) == golden['tokens_sha256']['idx']
    assert sha(targets) == golden['tokens_sha256']['targets']
    assert noise_sha(noise) == golden['noise_sha256']


def test_population_loss_matches_reference_at_init(golden, ref_inputs):
    _, params, _, idx, targets, noise, sign = ref_inputs
    losses = om.population_loss(params, noise, sign, idx, targets)
    assert torch.allclose(losses, torch.tensor(golden['losses_init']), atol=2e-6, rtol=0)


def test_population_loss_matches_reference_trained(golden, ref_inputs):
    model, _, _, idx, targets, noise, sign = ref_inputs
    m2 = trained_like(make_model('cpu', 0))
    for name, digest in golden['trained_weights_sha256'].items():
        assert sha(m2.state_dict()[name]) == digest, name
    params = {n: p.detach().clone() for n, p in m2.named_parameters()}
    losses = om.population_loss(params, noise, sign, idx, targets)
    ref = torch.tensor(golden['losses_trained'])
    assert torch.allclose(losses, ref, atol=2e-5, rtol=0)
    # the antithetic differences, which carry the ES signal, match too
    assert torch.allclose(losses[1::2] - losses[0::2], ref[1::2] - ref[0::2], atol=2e-5)


def test_clean_forward_matches_reference(golden, ref_inputs):
    model, params, _, idx, targets, _, _ = ref_inputs
    assert abs(float(om.gpt_forward(params, idx[None], targets[None])) - golden['clean_loss_init']) < 2e-6
    m2 = trained_like(make_model('cpu', 0))
    p2 = {n: p.detach().clone() for n, p in m2.named_parameters()}
    assert abs(float(om.gpt_forward(p2, idx[None], targets[None])) - golden['clean_loss_trained']) < 2e-5
    per_tok = om.gpt_forward(p2, idx[None], targets[None], loss_reduction='none')
    assert torch.allclose(per_tok, torch.tensor(golden['clean_token_losses_trained']), atol=5e-5)


def test_eggroll_step_matches_reference(golden):
    """Two whole `Eggroll.step` updates recomposed from the oracle's pieces: offsets, gathered noise,
    population losses, fitness, update and Adam (train/val/eggroll.py:117-168)."""
    st = golden['eggroll_step']
    model = trained_like(make_model('cpu', 0))
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    shapes = {n: tuple(p.shape) for n, p in params.items()}
    pairs, chunk, length = golden['pairs'], st['chunk'], st['noise_len']
    buf = oe.noise_buffer(length)
    assert sha(buf) == st['buffer_sha256']
    sx, sy = zipf_tokens(st['T'], seed=st['seq_seed'])
    state = {n: (torch.zeros_like(p), torch.zeros_like(p)) for n, p in params.items()}
    for rec in st['steps']:
        step = rec['step']
        offs = oe.offsets(shapes, pairs, step, length)
        for n in shapes:
            assert offs[n].tolist() == rec['offsets'][n], n
        dirs = oe.member_directions(0, chunk, pairs)
        gathered = oe.gather_noise(buf, offs, shapes, dirs)
        noise = {n: tuple(t.repeat_interleave(2, 0) for t in v) if isinstance(v, tuple) else v.repeat_interleave(2, 0)
                 for n, v in gathered.items()}
        sign = torch.tensor([oe.SIGMA, -oe.SIGMA]).repeat(chunk)
        losses = om.population_loss(params, noise, sign, sx, sy, cos=None)
        assert torch.allclose(losses, torch.tensor(rec['member_losses']), atol=3e-5), step
        assert abs(float(losses.mean()) - rec['mean_loss']) < 3e-5
        # fitness / update from the reference's losses so the comparison isolates these stages
        f, w = oe.fitness(torch.tensor(rec['member_losses']), pairs)
        grads = oe.update(w, oe.gather_noise(buf, offs, shapes, torch.arange(pairs)), len(f))
        for n, g in grads.items():
            ref = rec['grads'][n]
            if isinstance(ref, list):
                assert torch.allclose(g.flatten(), torch.tensor(ref), atol=1e-6, rtol=1e-4), n
            else:
                vals = torch.tensor([float(g[tuple(i)]) for i in ref['idx']])
                assert torch.allclose(vals, torch.tensor(ref['val']), atol=1e-7, rtol=1e-4), n
                assert float(g.double().abs().sum()) == pytest.approx(ref['abs_sum'], rel=1e-5)
        for n, p in params.items():
            before = p.clone()
            oe.adam_step(p, grads[n], *state[n], step, oe.LR)
            d = p - before
            ref = rec['deltas'][n]
            if isinstance(ref, list):
                assert torch.allclose(d.flatten(), torch.tensor(ref), atol=2e-9, rtol=1e-3), n
            else:
                vals = torch.tensor([float(d[tuple(i)]) for i in ref['idx']])
                assert torch.allclose(vals, torch.tensor(ref['val']), atol=2e-9, rtol=1e-3), n
