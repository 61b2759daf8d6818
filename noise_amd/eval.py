"""The speedrun's score on the HIP kernels: mean next-token cross-entropy of a state dict over a token
split (utils/eval.py:24-53).

`load_model` builds the fixed model from a strict state dict, as the reference does on a GPU, where
`init_weights` stores the token and value embeddings in bfloat16 before the state dict is copied in
(utils/model.py:171-175, utils/eval.py:24-31): the tables here keep fp32 storage holding the
bf16-rounded values, which is what the kernels read. `evaluate` runs `GPT.forward(..., 'sum')` over
batches of rows on the population kernels at sigma = 0 (head='bf16' by default; 'fp32' for the
fp32-accurate head), accumulates in fp64 and returns the mean over all predictions.

Rounding differs from utils/eval.py. The reference runs GPT.forward under CUDA autocast with bf16 embeddings, so
its whole residual stream is bf16: x0, every residual add and mix, the norms' outputs, rotary's products, the value
gate and the attention probabilities round to bf16 (rms_norm and the 0-dim lambda products keep their input's
bf16 dtype, and F.rms_norm's default eps follows the input dtype: 2^-7 for bf16). The kernels keep the population
path's rounding points instead: an fp32 residual stream and fp32 norms, bf16 GEMM operands and outputs, fp16
attention operands. On a trained-scale synthetic model (4 x 256 tokens, CPU) the two mean losses differ by 1.8e-3.
That is the size of the shift any single one of those rounding points produces on its own there (0.4e-3 to
2.0e-3 each: the bf16 stream, its eps, the bf16 tables, rotary's per-product rounding, bf16 q / k / P, the bf16
head), and of the shift the GEMMs' fp32 accumulation order alone produces at that scale (~1.5e-3), so a score from
`evaluate` agrees with the reference's to about 2e-3, not better.
"""
from pathlib import Path

import torch
from torch import distributed as dist

from .model import GPT, GPTConfig
from .population import Weights, clean_forward

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
def evaluate(state_dict, data_dir='data', batch_size=16, rows=None, head='bf16'):
    """Mean loss over every prediction of `rows` ([n, T + 1] token ids; by default the validation split
    under data_dir). Under torch.distributed the rows are split across ranks and the sums all-reduced."""
    rank, world = (dist.get_rank(), dist.get_world_size()) if dist.is_initialized() else (0, 1)
    device = torch.device('cuda', torch.cuda.current_device())
    model = load_model(state_dict, device)
    if rows is None:
        rows = load_rows(Path(data_dir) / 'val.pt')
    rows = rows[rank::world]
    weights = Weights(dict(model.named_parameters()), model.config, head)
    total = torch.zeros(2, dtype=torch.float64, device=device)  # summed loss, predictions
    for batch in rows.split(batch_size):
        batch = batch.to(device)
        loss = clean_forward(model, batch[:, :-1].contiguous(), batch[:, 1:].contiguous(), 'sum', head=head,
                             weights=weights)
        total[0] += loss.double()
        total[1] += batch[:, 1:].numel()
    if world > 1:
        dist.all_reduce(total)
    value = (total[0] / total[1]).item()
    if value != value:
        raise FloatingPointError('Non-finite validation loss')
    return value
