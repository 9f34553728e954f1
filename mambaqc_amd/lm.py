"""QuaternionMamba2 language model on MI355X: embedding -> N blocks -> LayerNorm -> head.

Drop-in for mambaqc/models/quaternion_mamba2.py:13-313: the same constructor,
padded vocabulary, module order and weight initialisation (so seeded weights
and state dicts are interchangeable), the same forward ({"logits", "loss"},
the same input assertions and cross-entropy), the same presets, and a
generate() with the same sampling rules.

generate() differs in cost, not in result: the reference re-runs the full
forward over the whole sequence for every new token
(quaternion_mamba2.py:192-225, O(T^2)); here the prompt runs once and each new
token is one recurrent step through every block, carrying the blocks' conv
tails and SSM states (QuaternionMamba2Block.forward_with_state).

The blocks run on the HIP kernels; embedding, LayerNorm, the head and the loss
are torch ops.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .block import QuaternionMamba2Block


class QuaternionMamba2(nn.Module):
    """Input [batch, seq_len] token ids -> {"logits": [batch, seq_len, vocab_size], "loss"}."""

    def __init__(self, vocab_size: int, d_model: int = 768, n_layers: int = 12,
                 d_state: int = 64, d_conv: int = 4, expand_factor: int = 2,
                 pad_vocab_size_multiple: int = 8, bias: bool = False, dropout: float = 0.0):
        super().__init__()
        self.vocab_size = vocab_size
        self.d_model = d_model
        self.n_layers = n_layers
        m = pad_vocab_size_multiple
        self.vocab_size_padded = (vocab_size + m - 1) // m * m if m > 1 else vocab_size

        # Module order fixes both the RNG stream and the apply() traversal of
        # the re-initialisation below (reference :60-88).
        self.embedding = nn.Embedding(self.vocab_size_padded, d_model)
        self.dropout = nn.Dropout(dropout) if dropout > 0.0 else nn.Identity()
        self.layers = nn.ModuleList([
            QuaternionMamba2Block(d_model=d_model, d_state=d_state, d_conv=d_conv,
                                  expand_factor=expand_factor, bias=bias)
            for _ in range(n_layers)
        ])
        self.norm_f = nn.LayerNorm(d_model)
        self.lm_head = nn.Linear(d_model, self.vocab_size_padded, bias=False)
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module: nn.Module) -> None:
        """N(0, 0.02) for nn.Linear / nn.Embedding weights, zero biases, unit
        LayerNorm (reference :90-100). The blocks' QuaternionLinear and conv
        weights are not nn.Linear and keep their own initialisation."""
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
        elif isinstance(module, nn.LayerNorm):
            nn.init.ones_(module.weight)
            nn.init.zeros_(module.bias)

    def _check_ids(self, input_ids: torch.Tensor) -> None:
        # Same checks as the reference (:122-124); they synchronise with the device.
        assert input_ids.min() >= 0, f"Negative token index: {input_ids.min().item()}"
        assert input_ids.max() < self.vocab_size, \
            f"Token index {input_ids.max().item()} >= vocab_size {self.vocab_size}"

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        return self.lm_head(self.norm_f(x))[..., : self.vocab_size]

    def forward(self, input_ids: torch.Tensor, labels: torch.Tensor | None = None):
        self._check_ids(input_ids)
        x = self.dropout(self.embedding(input_ids))
        for layer in self.layers:
            x = layer(x)
        logits = self._head(x)
        loss = None
        if labels is not None:
            valid = labels[labels != -100]
            if len(valid) > 0:
                assert valid.min() >= 0, f"Negative label: {valid.min().item()}"
                assert valid.max() < self.vocab_size, \
                    f"Label {valid.max().item()} >= vocab_size {self.vocab_size}"
            loss = nn.functional.cross_entropy(logits.reshape(-1, self.vocab_size),
                                               labels.reshape(-1), ignore_index=-100)
        return {"logits": logits, "loss": loss}

    def forward_with_state(self, input_ids: torch.Tensor, states=None):
        """Logits of input_ids continuing from per-layer recurrent states
        (None = start of sequence); returns (logits, new_states)."""
        self._check_ids(input_ids)
        return self._forward_with_state(input_ids, states)

    def _forward_with_state(self, input_ids: torch.Tensor, states=None):
        """forward_with_state without the id range check. The check reads the ids
        back to the host (two .item() calls), which stalls the host until the GPU
        has drained its queue; generate() feeds back tokens it sampled itself,
        which are in range by construction, so its decode steps skip it and the
        host stays ahead of the GPU."""
        x = self.dropout(self.embedding(input_ids))
        new_states = []
        for i, layer in enumerate(self.layers):
            x, st = layer.forward_with_state(x, None if states is None else states[i])
            new_states.append(st)
        return self._head(x), new_states

    def _step_state_(self, input_ids: torch.Tensor, states) -> torch.Tensor:
        """Logits [batch, 1, vocab] of one token per sequence continued from the
        per-layer states, which are updated in place (QuaternionMamba2Block.step_state_:
        contiguous conv tails in the model's dtype, fp32 SSM states). No id check,
        as in _forward_with_state."""
        x = self.dropout(self.embedding(input_ids))
        for layer, st in zip(self.layers, states):
            x = layer.step_state_(x, st)
        return self._head(x)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 100,
                 temperature: float = 1.0, top_k: int | None = None,
                 top_p: float | None = None, use_graph: bool = False) -> torch.Tensor:
        """Autoregressive sampling with the reference's rules (:169-227):
        temperature, then top-k, then nucleus (top-p) filtering, then one
        torch.multinomial draw per sequence per step.

        use_graph: run the decode steps as replays of one captured HIP graph
        (DecodeGraph) instead of launching every kernel from Python; the same
        kernels on the same data, so the same tokens."""
        self.eval()
        if max_new_tokens <= 0:
            return input_ids
        logits, states = self.forward_with_state(input_ids)
        graph = DecodeGraph(self, states) if use_graph and max_new_tokens > 1 else None
        # The decode steps update these states in place (contiguous tails: the
        # prompt's are views of its last rows).
        states = [(tail.contiguous(), h) for tail, h in states]
        for step in range(max_new_tokens):
            nxt = logits[:, -1, :] / temperature
            if top_k is not None:
                kth = torch.topk(nxt, top_k)[0][..., -1, None]
                nxt = nxt.masked_fill(nxt < kth, float("-inf"))
            if top_p is not None:
                sorted_logits, order = torch.sort(nxt, descending=True)
                cum = torch.cumsum(torch.softmax(sorted_logits, dim=-1), dim=-1)
                drop = cum > top_p
                # Keep the first token past the threshold as well.
                drop[..., 1:] = drop[..., :-1].clone()
                drop[..., 0] = False
                nxt = nxt.masked_fill(drop.scatter(1, order, drop), float("-inf"))
            token = torch.multinomial(torch.softmax(nxt, dim=-1), num_samples=1)
            input_ids = torch.cat([input_ids, token], dim=1)
            if step + 1 < max_new_tokens:
                if graph is not None:
                    logits = graph.step(token)
                else:
                    logits = self._step_state_(token, states)
        return input_ids

    def get_num_params(self, non_embedding: bool = True) -> int:
        """Parameter count, without the embedding and the (untied) head by default
        (reference :229-247)."""
        n = sum(p.numel() for p in self.parameters())
        if non_embedding:
            n -= self.embedding.weight.numel()
            if self.lm_head.weight is not self.embedding.weight:
                n -= self.lm_head.weight.numel()
        return n


class DecodeGraph:
    """One recurrent decode step of a QuaternionMamba2 (a token per sequence
    through every block) captured as a HIP graph, for serving loops where the
    step's ~12 kernels per layer would otherwise each be launched from Python.

    The graph reads its tokens and the per-layer states (conv tails, fp32 SSM
    states) from static buffers and its kernels update those states in place
    (QuaternionMamba2Block.step_state_), so each replay advances the sequences
    by one token: step(tokens) copies the
    tokens in, replays, and returns the static logits buffer [batch, 1, vocab]
    (valid until the next step). Built from the states a prompt's
    forward_with_state returned (they are copied; the caller's stay as they
    were). Capture follows torch's rules: warm-up steps on a side stream first
    (then the states are restored), and every intermediate tensor lives in the
    graph's memory pool. None of the library's kernels records a memset.

    The graph holds the device addresses it was captured with, including the
    fp32 copies of 16-bit parameters that the kernels read: build it once the
    weights are final, and build a new one after any weight update or
    .to()/.load_state_dict() on the model.
    """

    def __init__(self, lm: QuaternionMamba2, states, warmup: int = 2):
        dev = lm.embedding.weight.device
        batch = states[0][1].shape[0]
        self.lm = lm
        self.tokens = torch.zeros(batch, 1, dtype=torch.long, device=dev)
        self.states = [(tail.detach().clone(memory_format=torch.contiguous_format),
                        h.detach().clone(memory_format=torch.contiguous_format))
                       for tail, h in states]
        saved = [(tail.clone(), h.clone()) for tail, h in self.states]
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._step()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._step()
        for (tail, h), (t0, h0) in zip(self.states, saved):
            tail.copy_(t0)
            h.copy_(h0)

    def _step(self) -> torch.Tensor:
        return self.lm._step_state_(self.tokens, self.states)

    def step(self, tokens: torch.Tensor) -> torch.Tensor:
        self.tokens.copy_(tokens)
        self.graph.replay()
        return self.logits


def quaternion_mamba2_small(vocab_size: int) -> QuaternionMamba2:
    """d_model 512, 8 layers, d_state 32 (reference :286-293)."""
    return QuaternionMamba2(vocab_size=vocab_size, d_model=512, n_layers=8, d_state=32)


def quaternion_mamba2_base(vocab_size: int) -> QuaternionMamba2:
    """d_model 768, 12 layers, d_state 64 (reference :296-303). With the
    reference's B/C projections this is 14.66 B parameters (29.3 GB in bf16),
    not the ~150M its docstring says."""
    return QuaternionMamba2(vocab_size=vocab_size, d_model=768, n_layers=12, d_state=64)


def quaternion_mamba2_large(vocab_size: int) -> QuaternionMamba2:
    """d_model 1024, 24 layers, d_state 64 (reference :306-313)."""
    return QuaternionMamba2(vocab_size=vocab_size, d_model=1024, n_layers=24, d_state=64)
