"""Host side of the score (noise_amd.eval, utils/eval.py:24-53): strict state-dict loading and the split
format, on the CPU."""
import pytest
import torch

from noise_amd.eval import SEQ, load_model, load_rows
from noise_amd.model import make_model


def test_load_model_is_strict_and_keeps_the_weights():
    sd = make_model('cpu', 0).state_dict()
    m = load_model(sd, 'cpu')
    assert all(torch.equal(m.state_dict()[k], v) for k, v in sd.items())
    missing = dict(sd)
    missing.pop('lm_head.weight')
    with pytest.raises(RuntimeError):
        load_model(missing, 'cpu')
    extra = dict(sd, bogus=torch.zeros(1))
    with pytest.raises(RuntimeError):
        load_model(extra, 'cpu')
    reshaped = dict(sd, **{'lm_head.weight': torch.zeros(4096, 256)})
    with pytest.raises(RuntimeError):
        load_model(reshaped, 'cpu')


def test_load_rows_checks_the_split_shape(tmp_path):
    good = torch.randint(0, 4096, (3, SEQ), dtype=torch.int32)
    torch.save(good, tmp_path / 'val.pt')
    assert torch.equal(load_rows(tmp_path / 'val.pt', 3), good.long())
    with pytest.raises(ValueError):
        load_rows(tmp_path / 'val.pt', 4)
    torch.save(torch.zeros(3, SEQ - 1, dtype=torch.int32), tmp_path / 'bad.pt')
    with pytest.raises(ValueError):
        load_rows(tmp_path / 'bad.pt', 3)
