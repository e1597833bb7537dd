"""Autoregressive generation (mamba_metal/generate.py:16-110).

  generate       O(L^2): re-runs the full forward for every new token (the
                 reference's correctness baseline, generate.py:16-62).
  generate_fast  one parallel prefill, then O(1) ``model.step`` per token
                 (generate.py:65-110).  Same signature and string semantics:
                 greedy when temperature == 0, else sampling from softmax(logits/T);
                 stops at the tokenizer's EOS; ``on_token`` streams text deltas.

Token-level API for serving and benchmarks (no tokenizer, batch > 1, no EOS):
  generate_fast_ids  prefill + decode on token ids, greedy or sampled.
  GraphDecoder       the decode step (embedding -> layers -> head -> argmax)
                     captured once into a HIP graph and replayed per token, with
                     the resident conv/SSM states updated in place; its prefill
                     replayed from a GraphPrefill.
  GraphPrefill       MambaModel.prefill captured once per prompt shape (batch,
                     seqlen) into a HIP graph and replayed: the per-op host dispatch
                     of the layer loop (~10 ops per layer) is paid once, at capture.
"""

from __future__ import annotations

from typing import Callable

import torch

from mamba_metal_amd.sample import argmax_rows


def _argmax(logits: torch.Tensor) -> torch.Tensor:
    """Greedy ids over the last axis on the library kernel (rows flattened)."""
    flat = logits.reshape(-1, logits.shape[-1]) if logits.stride(-1) == 1 else \
        logits.contiguous().reshape(-1, logits.shape[-1])
    return argmax_rows(flat).reshape(logits.shape[:-1])


def _sample(logits: torch.Tensor, temperature: float, generator=None) -> torch.Tensor:
    if temperature == 0.0:
        return _argmax(logits)
    probs = torch.softmax(logits.float() / temperature, dim=-1)
    return torch.multinomial(probs, 1, generator=generator).squeeze(-1)


def _encode(tokenizer, prompt: str, device) -> torch.Tensor:
    ids = tokenizer(prompt, return_tensors="np").input_ids
    return torch.as_tensor(ids, dtype=torch.long, device=device)


def _stream(tokenizer, prompt, generated_ids, prev_text, on_token):
    new_text = tokenizer.decode(generated_ids, skip_special_tokens=True)
    delta = new_text[len(prev_text) - len(prompt):]
    if delta:
        on_token(delta)
        return prompt + new_text
    return prev_text


@torch.inference_mode()
def generate(model, tokenizer, prompt: str, max_new_tokens: int = 50, temperature: float = 0.0,
             on_token: Callable[[str], None] | None = None) -> str:
    """O(L^2) generation: full forward over the whole prefix for each token."""
    device = model.embeddings.weight.device
    input_ids = _encode(tokenizer, prompt, device)
    eos = tokenizer.eos_token_id
    generated_ids: list[int] = []
    prev_text = prompt
    for _ in range(max_new_tokens):
        next_logits = model(input_ids)[:, -1, :]
        next_id = _sample(next_logits, temperature)
        next_id_int = int(next_id.reshape(-1)[0].item())
        if eos is not None and next_id_int == eos:
            break
        generated_ids.append(next_id_int)
        if on_token is not None:
            prev_text = _stream(tokenizer, prompt, generated_ids, prev_text, on_token)
        input_ids = torch.cat([input_ids, next_id.reshape(1, 1).to(input_ids.dtype)], dim=1)
    return prompt + tokenizer.decode(generated_ids, skip_special_tokens=True)


@torch.inference_mode()
def generate_fast(model, tokenizer, prompt: str, max_new_tokens: int = 50,
                  temperature: float = 0.0,
                  on_token: Callable[[str], None] | None = None) -> str:
    """O(L_prompt + n_decode) generation: parallel prefill, then O(1) steps."""
    device = model.embeddings.weight.device
    input_ids = _encode(tokenizer, prompt, device)
    eos = tokenizer.eos_token_id
    logits, conv_states, ssm_states = model.prefill(input_ids, last_only=True)
    next_logits = logits[:, -1, :]
    generated_ids: list[int] = []
    prev_text = prompt
    for _ in range(max_new_tokens):
        next_id = _sample(next_logits, temperature)
        next_id_int = int(next_id.reshape(-1)[0].item())
        if eos is not None and next_id_int == eos:
            break
        generated_ids.append(next_id_int)
        if on_token is not None:
            prev_text = _stream(tokenizer, prompt, generated_ids, prev_text, on_token)
        ids = torch.tensor([[next_id_int]], dtype=torch.long, device=device)
        step_logits, conv_states, ssm_states = model.step(ids, conv_states, ssm_states,
                                                          inplace=True)
        next_logits = step_logits[:, 0, :]
    return prompt + tokenizer.decode(generated_ids, skip_special_tokens=True)


class GraphPrefill:
    """``MambaModel.prefill(input_ids, last_only=True)`` replayed from a HIP graph
    captured once per ``(batch, seqlen)``.

    Calling it copies ``input_ids`` into the graph's input buffer, replays the graph and
    returns ``(logits (B, 1, vocab), conv_states, ssm_states)`` -- tensors owned by that
    shape's graph: the same tensors come back from every call of that shape and are
    overwritten by the next one (copy what must outlive it).  The captured graph runs the
    same kernels in the same order as the eager prefill (its results are identical); it
    holds its own memory pool per captured shape (``clear()`` releases them)."""

    def __init__(self, model):
        self.model = model
        self._graphs: dict = {}

    def clear(self) -> None:
        self._graphs.clear()

    def _capture(self, input_ids):
        ids = input_ids.clone()
        # Warm up on a side stream first (lazy library init, hipBLASLt heuristics for these
        # shapes); capturing does not execute anything.
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.model.prefill(ids, last_only=True)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            logits, convs, ssms = self.model.prefill(ids, last_only=True)
        ent = (g, ids, logits, convs, ssms)
        self._graphs[tuple(input_ids.shape)] = ent
        return ent

    @torch.inference_mode()
    def __call__(self, input_ids: torch.Tensor):
        ent = self._graphs.get(tuple(input_ids.shape))
        if ent is None:
            ent = self._capture(input_ids)
        g, ids, logits, convs, ssms = ent
        ids.copy_(input_ids)
        g.replay()
        return logits, convs, ssms


class GraphDecoder:
    """Greedy/sampled decode with the whole step captured in one HIP graph.

    ``start(input_ids)`` runs the parallel prefill (its states become the resident
    decode state) and returns the first token; ``step()`` replays the captured
    graph -- embedding, every layer's in-place conv/SSM update, the head and
    argmax -- and returns the next token ids (B,) on the device, with no host
    sync.  Greedy only when captured (``temperature == 0``); sampling runs eagerly.
    With ``use_graph`` the prefill is replayed from a ``GraphPrefill`` as well: the
    resident decode state is then the captured prefill's own state buffers for the
    first prompt shape (a later prompt of that shape writes its state into them
    directly; other shapes are copied in).

    ``steps_per_graph`` = K > 1 captures K consecutive steps in one graph (each replay
    boundary costs ~5 µs on MI355X, 2% of a Mamba-130M batch-1 step): a replay runs K
    steps, ``step()`` hands their ids out one per call (the same ids, in the same order,
    as K = 1), and the resident state runs up to K - 1 steps ahead of the ids returned.
    The K steps pass their ids through a ring of K rows: step j reads row j - 1 (mod K)
    and its argmax writes row j.  The embedding row of the next step's ids is written by
    the same kernel that picks them (``step_greedy(hidden=...)``), so no step runs an
    embedding lookup of its own.
    """

    def __init__(self, model, batch_size: int, use_graph: bool = True, steps_per_graph: int = 1):
        self.model = model
        self.batch = batch_size
        self.use_graph = use_graph
        self.k = max(1, int(steps_per_graph)) if use_graph else 1
        self.graph = None
        self.ids = None
        self.ring = None     # (K, B) ids of one replay (K > 1)
        self.hid = None      # (B, d_model) embedding rows of the next step's input ids
        self.pending = 0     # ids of the last replay not yet handed out
        self.convs = None
        self.ssms = None
        self.prefill = GraphPrefill(model) if use_graph else None

    def _step_into(self, src, dst):
        """One decode step on input ids ``src``; its greedy ids go to ``dst`` (which may be
        ``src``: the embedding reads it before the argmax writes).  The head and the
        argmax run as one call (``MambaModel.step_greedy``)."""
        self.model.step_greedy(src.view(-1, 1), self.convs, self.ssms, dst, hidden=self.hid)
        return dst

    def _eager_step(self):
        """One decode step whose greedy ids overwrite ``self.ids``."""
        return self._step_into(self.ids, self.ids)

    def _graph_steps(self):
        """What one replay runs: one step in place, or K steps through the id ring."""
        if self.k == 1:
            self._eager_step()
            return
        for j in range(self.k):
            self._step_into(self.ring[(j - 1) % self.k], self.ring[j])

    @torch.inference_mode()
    def start(self, input_ids: torch.Tensor) -> torch.Tensor:
        assert input_ids.shape[0] == self.batch
        if self.prefill is not None:
            logits, convs, ssms = self.prefill(input_ids)
        else:
            logits, convs, ssms = self.model.prefill(input_ids, last_only=True)
        first = _argmax(logits[:, -1, :])
        if self.convs is None:
            self.convs, self.ssms = list(convs), list(ssms)
            self.ids = first.clone()
            if self.k > 1:
                self.ring = torch.empty((self.k,) + tuple(first.shape), dtype=first.dtype,
                                        device=first.device)
        else:  # keep the captured buffers; copy the new prefill state into them
            for dst, src in zip(self.convs + self.ssms, list(convs) + list(ssms)):
                if dst is not src:
                    dst.copy_(src)
            self.ids.copy_(first)
        if self.ring is not None:
            self.ring[self.k - 1].copy_(first)  # the next replay's first input
            self.pending = 0
        rows = self.model.embeddings(first)
        if self.hid is None:
            self.hid = rows
        else:
            self.hid.copy_(rows)
        if self.use_graph and self.graph is None:
            self._capture()
        return first

    def _capture(self):
        # Warm up on a side stream (lazy library init, hipBLASLt heuristics), then
        # restore the state the warm-up step advanced.
        bufs = self.convs + self.ssms + [self.ids, self.hid] + \
            ([self.ring] if self.ring is not None else [])
        saved = [t.clone() for t in bufs]
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._graph_steps()
        torch.cuda.current_stream().wait_stream(s)
        for dst, src in zip(bufs, saved):
            dst.copy_(src)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._graph_steps()  # the argmax writes the next step's input ids in place
        # Capturing does not execute; the state is still the prefill state.
        self.graph = g

    @torch.inference_mode()
    def step(self) -> torch.Tensor:
        """Advance every sequence by one token; returns the next ids (B,).

        The returned tensor is one of the decoder's own id buffers, which a later step
        overwrites (clone what must be kept)."""
        if self.graph is None:
            return self._eager_step()
        if self.k == 1:
            self.graph.replay()
            return self.ids
        if self.pending == 0:
            self.graph.replay()
            self.pending = self.k
        j = self.k - self.pending
        self.pending -= 1
        return self.ring[j]


@torch.inference_mode()
def generate_fast_ids(model, input_ids: torch.Tensor, max_new_tokens: int,
                      temperature: float = 0.0, eos_token_id: int | None = None,
                      generator: torch.Generator | None = None,
                      use_graph: bool = False) -> torch.Tensor:
    """Token-id generate_fast for a (B, L) batch.  Returns (B, max_new_tokens) ids.

    Greedy when temperature == 0.  With eos_token_id set (batch 1 only), stops at
    EOS as the reference does and returns the ids before it.  use_graph replays
    a captured HIP graph per step (greedy, no EOS)."""
    B = input_ids.shape[0]
    if max_new_tokens <= 0:
        return torch.empty((B, 0), dtype=torch.long, device=input_ids.device)
    if use_graph and temperature == 0.0 and eos_token_id is None:
        # several steps per replay where they divide the steps after the first token
        k = next(d for d in (8, 4, 2, 1) if (max_new_tokens - 1) % d == 0) if max_new_tokens > 1 else 1
        dec = GraphDecoder(model, B, use_graph=True, steps_per_graph=k)
        toks = [dec.start(input_ids).clone()]
        for _ in range(max_new_tokens - 1):
            toks.append(dec.step().clone())
        return torch.stack(toks[:max_new_tokens], dim=1)
    logits, convs, ssms = model.prefill(input_ids, last_only=True)
    nxt = logits[:, -1, :]
    out = []
    for i in range(max_new_tokens):
        tok = _sample(nxt, temperature, generator)
        if eos_token_id is not None and B == 1 and int(tok[0].item()) == eos_token_id:
            break
        out.append(tok)
        if i + 1 == max_new_tokens:
            break
        step_logits, convs, ssms = model.step(tok.view(-1, 1), convs, ssms, inplace=True)
        nxt = step_logits[:, 0, :]
    if not out:
        return torch.empty((B, 0), dtype=torch.long, device=input_ids.device)
    return torch.stack(out, dim=1)
