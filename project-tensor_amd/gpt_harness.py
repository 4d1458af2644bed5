"""GPT-style training step composed from the tensor_gpu_v2 API.

Pre-LayerNorm decoder: tied token embedding, per layer LN -> one Q/K/V Linear(d, 3d)
-> causal FlashAttention on the packed projection (flash_attention_qkv: q, k and v
read in place, the heads merged on output) -> O Linear -> residual, LN ->
Linear(d, 4d) -> GELU -> Linear(4d, d) -> residual; final LN; logits = h @ E^T; CrossEntropyLoss.  The residual adds and the
GELU run in the adjacent Linear GEMMs' epilogues (Linear's residual= / activation=
options: the same graph and values as the separate ops).  One step runs the forward
under fp16 autocast, GradScaler.scale(loss).backward(), sync_tied_gradients,
unscale_, clip_grad_norm_(1.0), GradScaler.step(AdamW) and update().

The reference has no GPT model class on the gradient path; this harness builds the
configuration from the same public primitives a reference user would combine
(Embedding, Linear, LayerNorm, flash_attention(_qkv), CrossEntropyLoss, weight_tie,
sync_tied_gradients, AdamW, GradScaler, clip_grad_norm_).
"""
import gc

import numpy as np

import tensor_gpu_v2 as tg


def _normal(shape, std, rng):
    return (rng.standard_normal(shape) * std).astype(np.float32)


class Block(tg.Module):
    def __init__(self, d, heads, rng):
        super().__init__()
        self.d, self.heads = d, heads
        self.ln1 = tg.LayerNorm(d)
        self.ln2 = tg.LayerNorm(d)
        self.qkv = tg.Linear(d, 3 * d)  # columns: query heads | key heads | value heads
        self.o = tg.Linear(d, d)
        self.fc1 = tg.Linear(d, 4 * d)
        self.fc2 = tg.Linear(4 * d, d)
        for lin in (self.qkv, self.o, self.fc1, self.fc2):
            lin.w.data = tg.Tensor(_normal(lin.w.shape, 0.02, rng), requires_grad=False).data

    def __call__(self, h):
        att = tg.flash_attention_qkv(self.qkv(self.ln1(h)), self.heads, is_causal=True)
        # h + o(att) and fc2(gelu(fc1(m))) + h with the add and the GELU in the GEMMs'
        # epilogues (Linear's keyword options; the same ops, values and gradients)
        h = self.o(att, residual=h)
        m = self.ln2(h)
        return self.fc2(self.fc1(m, activation="gelu"), residual=h)


class GPT(tg.Module):
    def __init__(self, vocab=32000, d=1024, heads=16, layers=4, seed=0):
        super().__init__()
        rng = np.random.default_rng(seed)
        self.embed = tg.Embedding(vocab, d)
        self.embed.weight.data = tg.Tensor(_normal((vocab, d), 0.02, rng),
                                           requires_grad=False).data
        self.blocks = [Block(d, heads, rng) for _ in range(layers)]
        self.lnf = tg.LayerNorm(d)
        self.head = tg.Linear(d, vocab, bias=False)
        tg.weight_tie(self.embed.weight, self.head, "w", transpose=True)
        self.vocab = vocab

    def __call__(self, ids):
        h = self.embed(ids)
        for blk in self.blocks:
            h = blk(h)
        h = self.lnf(h)
        B, T, C = h.shape
        return self.head(h).reshape(B * T, self.vocab)


class Trainer:
    """One optimizer step per call: the C5 recipe (AdamW lr 3e-4, wd 0.1, clip 1.0,
    GradScaler init 2^16, fp16 autocast)."""

    def __init__(self, model, lr=3e-4, weight_decay=0.1, clip=1.0, init_scale=2.0 ** 16,
                 strict_chain_rule=False):
        self.model = model
        params = model.parameters()
        # every parameter, the tied head weight included (its gradient is transferred
        # to the embedding each step and must start from zero): the module tree is
        # fixed, so it is walked once here rather than per step
        self._all = params
        # the tied head weight is a view of the embedding: optimise the source only
        self.params = [p for p in params if not _is_tied(p)]
        self.opt = tg.AdamW(self.params, lr=lr, weight_decay=weight_decay)
        self.scaler = tg.GradScaler(init_scale=init_scale)
        self.clip = clip
        self.loss_fn = tg.CrossEntropyLoss(strict_chain_rule=strict_chain_rule)
        # Everything alive now (imported modules, the model, the optimizer state) is
        # long-lived: moved out of the cyclic collector's generations, the full
        # collections that each step's graph objects trigger every couple of dozen
        # steps stay short (traversing torch's ~170 K objects took ≈ 50 ms, one step in
        # ~25 at 8x the normal step time).
        gc.freeze()

    def step(self, ids, targets):
        for p in self._all:
            p.zero_grad()
        with tg.autocast():
            logits = self.model(ids)
            loss = self.loss_fn(logits, targets)
        self.scaler.scale(loss).backward()
        tg.sync_tied_gradients(self.model)
        self.scaler.unscale_(self.opt)
        norm = tg.clip_grad_norm_(self.params, self.clip)
        self.scaler.step(self.opt)
        self.scaler.update()
        return loss, norm


def _is_tied(p):
    try:
        return p._tied_source is not None
    except AttributeError:
        return False


def synthetic_batch(vocab=32000, batch=8, seq=1024, seed=0):
    """Uniform random token ids (inputs) and next-token targets."""
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, size=(batch, seq + 1))
    return ids[:, :-1].copy(), ids[:, 1:].reshape(-1).copy()
