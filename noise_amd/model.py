"""The fixed 37.7M GPT as a weight container with the reference's strict state dict.

The module tree (names, shapes, parameter order) is the contract `utils/eval.py:24-31` loads with
`strict=True`, so it is kept identical to `utils/model.py:61-147`. Compute never runs through these
nn.Modules: `GPT.forward` dispatches to the population kernels with one member per batch row and
sigma = 0 (`noise_amd.population.clean_forward`, or `autocast_forward` under torch's bf16 autocast).
"""
from dataclasses import dataclass

import torch
from torch import nn


@dataclass
class GPTConfig:
    """Model dims (utils/model.py:34-43)."""
    sequence_len: int = 2048
    vocab_size: int = 4096
    n_layer: int = 8
    n_head: int = 8
    n_kv_head: int = 8
    n_embd: int = 512
    window_pattern: str = 'SSSL'


VE_GATE_CHANNELS = 32  # utils/model.py:75


def has_ve(layer_idx, n_layer):
    """Value embeddings on every other block, counting back from the last (utils/model.py:50-52)."""
    return layer_idx % 2 == (n_layer - 1) % 2


def window_sizes(config):
    """Per-layer left window (utils/model.py:185-191), from config.sequence_len, not the runtime T."""
    pattern = config.window_pattern.upper()
    long_w, short_w = config.sequence_len, config.sequence_len // 2
    sizes = [long_w if pattern[i % len(pattern)] == 'L' else short_w for i in range(config.n_layer)]
    sizes[-1] = long_w
    return sizes


def rotary_tables(seq_len, head_dim, device=None, base=10000):
    """bf16 cos/sin [seq_len, head_dim // 2] (utils/model.py:177-183), computed on the CPU in fp32."""
    inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    cos, sin = freqs.cos().bfloat16(), freqs.sin().bfloat16()
    return cos.to(device), sin.to(device)


class CausalSelfAttention(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        d = config.n_embd
        kv = config.n_kv_head * (d // config.n_head)
        self.c_q = nn.Linear(d, d, bias=False)
        self.c_k = nn.Linear(d, kv, bias=False)
        self.c_v = nn.Linear(d, kv, bias=False)
        self.c_proj = nn.Linear(d, d, bias=False)
        self.ve_gate = (nn.Linear(VE_GATE_CHANNELS, config.n_kv_head, bias=False)
                        if has_ve(layer_idx, config.n_layer) else None)


class MLP(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.c_fc = nn.Linear(config.n_embd, 4 * config.n_embd, bias=False)
        self.c_proj = nn.Linear(4 * config.n_embd, config.n_embd, bias=False)


class Block(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        self.attn = CausalSelfAttention(config, layer_idx)
        self.mlp = MLP(config)


class GPT(nn.Module):
    """Parameter container with the state dict of `utils/model.py:123-147`."""

    def __init__(self, config=None, pad_vocab_size_to=64):
        super().__init__()
        config = config or GPTConfig()
        self.config = config
        self.window_sizes = [(w, 0) for w in window_sizes(config)]
        padded = (config.vocab_size + pad_vocab_size_to - 1) // pad_vocab_size_to * pad_vocab_size_to
        self.transformer = nn.ModuleDict({
            'wte': nn.Embedding(padded, config.n_embd),
            'h': nn.ModuleList([Block(config, i) for i in range(config.n_layer)]),
        })
        self.lm_head = nn.Linear(config.n_embd, padded, bias=False)
        self.resid_lambdas = nn.Parameter(torch.ones(config.n_layer))
        self.x0_lambdas = nn.Parameter(torch.zeros(config.n_layer))
        kv_dim = config.n_kv_head * (config.n_embd // config.n_head)
        self.value_embeds = nn.ModuleDict({
            str(i): nn.Embedding(padded, kv_dim) for i in range(config.n_layer) if has_ve(i, config.n_layer)
        })
        self.rotary_seq_len = config.sequence_len * 10
        head_dim = config.n_embd // config.n_head
        cos, sin = rotary_tables(self.rotary_seq_len, head_dim)
        self.register_buffer('cos', cos[None, :, None, :], persistent=False)
        self.register_buffer('sin', sin[None, :, None, :], persistent=False)

    @torch.no_grad()
    def init_weights(self):
        """Seeded init; the order of RNG draws is that of utils/model.py:150-175, so the CPU generator
        yields the reference's weights bit for bit."""
        cfg = self.config
        torch.nn.init.normal_(self.transformer.wte.weight, mean=0.0, std=1.0)
        torch.nn.init.normal_(self.lm_head.weight, mean=0.0, std=0.001)
        s = 3 ** 0.5 * cfg.n_embd ** (-0.5)
        for block in self.transformer.h:
            torch.nn.init.uniform_(block.attn.c_q.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_k.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_v.weight, -s, s)
            torch.nn.init.zeros_(block.attn.c_proj.weight)
            torch.nn.init.uniform_(block.mlp.c_fc.weight, -s, s)
            torch.nn.init.zeros_(block.mlp.c_proj.weight)
        self.resid_lambdas.fill_(1.0)
        self.x0_lambdas.fill_(0.1)
        for ve in self.value_embeds.values():
            torch.nn.init.uniform_(ve.weight, -s, s)
        for block in self.transformer.h:
            if block.attn.ve_gate is not None:
                torch.nn.init.zeros_(block.attn.ve_gate.weight)
        head_dim = cfg.n_embd // cfg.n_head
        cos, sin = rotary_tables(self.rotary_seq_len, head_dim, self.cos.device)
        self.cos, self.sin = cos[None, :, None, :], sin[None, :, None, :]

    def forward(self, idx, targets=None, loss_reduction='mean'):
        """Clean forward (utils/model.py:193-210) on the HIP kernels: one member per batch row, sigma = 0. Called
        under torch.autocast('cuda', dtype=torch.bfloat16), as utils/eval.py:44-45 calls it, it keeps that autocast's
        rounding points (noise_amd.population.autocast_forward); otherwise the population path's."""
        from .population import autocast_forward, clean_forward
        if torch.is_autocast_enabled('cuda') and torch.get_autocast_dtype('cuda') == torch.bfloat16:
            return autocast_forward(self, idx, targets, loss_reduction)
        return clean_forward(self, idx, targets, loss_reduction)


def make_model(device, seed=0, config=None):
    """EGGROLL's initialisation (train/val/eggroll.py:38-53): the Dust init, c_proj re-drawn
    U(+-1.5 sqrt(3 / fan_in)), embeddings float32, no grad.

    The weights are always drawn from the CPU generator, then moved, so every device gets the
    reference's `make_model('cpu', seed)` values. On a GPU the reference stores the embeddings in bf16
    inside init_weights (utils/model.py:171-175) before casting back to fp32; that rounding is kept."""
    torch.manual_seed(seed)
    with torch.device('meta'):
        model = GPT(config or GPTConfig())
    model.to_empty(device='cpu')
    model.init_weights()
    with torch.no_grad():
        for name, module in model.named_modules():
            if 'c_proj' in name and isinstance(module, nn.Linear):
                scale = 1.5 * (3 / module.weight.shape[1]) ** 0.5
                torch.nn.init.uniform_(module.weight, -scale, scale)
        if torch.device(device).type == 'cuda':
            for emb in [model.transformer.wte, *model.value_embeds.values()]:
                emb.weight.copy_(emb.weight.bfloat16().float())
    model.to(device)
    return model.requires_grad_(False)


def matrix_shapes(model):
    """name -> shape for every parameter in named_parameters order (the perturbation layout)."""
    return {name: tuple(p.shape) for name, p in model.named_parameters()}
