"""The speedrun's score on the HIP kernels: mean next-token cross-entropy of a state dict over a token
split (utils/eval.py:24-53).

`load_model` builds the fixed model from a strict state dict, as the reference does on a GPU, where
`init_weights` stores the token and value embeddings in bfloat16 before the state dict is copied in
(utils/model.py:171-175, utils/eval.py:24-31): the tables here keep fp32 storage holding the
bf16-rounded values, which is what the kernels read. `evaluate` runs `GPT.forward(..., 'sum')` over
batches of rows, accumulates in fp64 and returns the mean over all predictions.

Rounding. By default (`rounding='autocast'`) the forward keeps the rounding points utils/eval.py:44-45 gives it:
torch's bf16 autocast, under which the whole residual stream is bf16 and every op rounds to bf16 (x0, the lambda
mix with bf16-cast lambdas, the residual adds, the norms' outputs, rotary's products and sums, the value gate, bf16
q / k / v and probabilities in attention, the bf16 head); `noise_amd.population.autocast_forward` runs it and
`oracle.model.autocast_forward` restates it. `rounding='population'` runs the population path's rounding instead
(fp32 residual stream and norms, fp16 attention operands; head='bf16' or 'fp32'), which moves the score of a
trained-scale model by about 2e-3.
"""
from pathlib import Path

import torch
from torch import distributed as dist

from .model import GPT, GPTConfig
from .population import ROUNDINGS, Weights, autocast_forward, clean_forward

SEQ = 2049       # tokens per row: 2048 inputs + the shifted targets (utils/prepare_data.py:19)
VAL_ROWS = 544   # rows of the validation split, 1,114,112 predictions (utils/prepare_data.py:21)


def load_model(state_dict, device):
    """The fixed architecture with these weights; a missing, extra or reshaped tensor is an error
    (utils/eval.py:24-31)."""
    with torch.device('meta'):
        model = GPT(GPTConfig())
    model.to_empty(device=device)
    model.init_weights()
    model.load_state_dict(state_dict, strict=True)
    if torch.device(device).type == 'cuda':
        with torch.no_grad():
            for emb in [model.transformer.wte, *model.value_embeds.values()]:
                emb.weight.copy_(emb.weight.bfloat16().float())
    return model.eval().requires_grad_(False)


def load_rows(path, rows=VAL_ROWS):
    """A fixed split as int64 [rows, 2049] (utils/prepare_data.py:39-47, without the pinned-hash check:
    the reference's data files are not part of this build)."""
    data = torch.load(path, map_location='cpu', weights_only=True)
    if not isinstance(data, torch.Tensor) or tuple(data.shape) != (rows, SEQ):
        raise ValueError(f'{path}: expected a [{rows}, {SEQ}] token tensor')
    return data.long()


@torch.no_grad()
def evaluate(state_dict, data_dir='data', batch_size=16, rows=None, head='bf16', rounding='autocast'):
    """Mean loss over every prediction of `rows` ([n, T + 1] token ids; by default the validation split
    under data_dir). Under torch.distributed the rows are split across ranks and the sums all-reduced.
    rounding: 'autocast' (utils/eval.py's, the default) or 'population' (with `head`)."""
    if rounding not in ROUNDINGS:
        raise ValueError(f'rounding must be one of {ROUNDINGS}')
    rank, world = (dist.get_rank(), dist.get_world_size()) if dist.is_initialized() else (0, 1)
    device = torch.device('cuda', torch.cuda.current_device())
    model = load_model(state_dict, device)
    if rows is None:
        rows = load_rows(Path(data_dir) / 'val.pt')
    rows = rows[rank::world]
    weights = Weights(dict(model.named_parameters()), model.config, 'bf16' if rounding == 'autocast' else head)
    total = torch.zeros(2, dtype=torch.float64, device=device)  # summed loss, predictions
    for batch in rows.split(batch_size):
        batch = batch.to(device)
        x, y = batch[:, :-1].contiguous(), batch[:, 1:].contiguous()
        if rounding == 'autocast':
            loss = autocast_forward(model, x, y, 'sum', weights=weights)
        else:
            loss = clean_forward(model, x, y, 'sum', head=head, weights=weights)
        total[0] += loss.double()
        total[1] += batch[:, 1:].numel()
    if world > 1:
        dist.all_reduce(total)
    value = (total[0] / total[1]).item()
    if value != value:
        raise FloatingPointError('Non-finite validation loss')
    return value
