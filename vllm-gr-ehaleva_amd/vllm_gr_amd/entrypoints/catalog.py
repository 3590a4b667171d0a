"""Catalog of valid semantic-ID token sequences.

``Catalog`` keeps the reference's interface (vllm_gr/entrypoints/openai/
serving_models.py:18-49): ``load(path)`` reads a JSON list of token-string
sequences through the tokenizer's ``convert_tokens_to_ids`` into a trie, and
``valid(token_ids)`` returns the tokens that may follow a generated prefix
(the empty set once the prefix leaves the trie).  ``add`` takes token ids
directly (there is no tokenizer here).

``to_device`` lays the trie out for gr_beam_prune_topk_catalog: nodes
numbered in breadth-first order from the root (node 0), each node's children
contiguous and ascending by token -- ``node_start [nodes + 1]``,
``child_token [edges]``, ``child_node [edges]`` (int32).  A beam then carries
one node id instead of its token history; ``node_of(token_ids)`` gives the
id the device walk reaches (-1 when the prefix leaves the trie).
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from typing import Any

import torch


@dataclass
class CatalogTensors:
    node_start: torch.Tensor   # [num_nodes + 1] int32
    child_token: torch.Tensor  # [num_edges] int32
    child_node: torch.Tensor   # [num_edges] int32

    @property
    def num_nodes(self) -> int:
        return self.node_start.numel() - 1

    @property
    def num_edges(self) -> int:
        return self.child_token.numel()


class Catalog:
    def __init__(self, tokenizer=None):
        self.tokenizer = tokenizer
        self.trie: dict[int, Any] = {}
        self._csr = None
        self._ids = None

    def load(self, path: str) -> None:
        try:
            with open(path) as f:
                data = json.load(f)
        except FileNotFoundError:
            raise ValueError(f"Catalog file not found: {path}") from None
        except json.JSONDecodeError:
            raise ValueError(f"Failed to decode JSON from catalog file: {path}") from None
        if self.tokenizer is None:
            raise ValueError("loading token strings needs a tokenizer; use add() with token ids")
        for seq in data:
            ids = self.tokenizer.convert_tokens_to_ids(seq)
            for i, t in enumerate(ids):
                if t is None:
                    raise ValueError(f"Invalid token ID: {seq[i]} at index {i}")
            self.add(ids)

    def add(self, token_ids) -> None:
        node = self.trie
        for t in token_ids:
            node = node.setdefault(int(t), {})
        self._csr = None

    def valid(self, token_ids) -> set[int]:
        node = self.trie
        for t in token_ids:
            if t in node:
                node = node[t]
            else:
                return set()
        return set(node.keys())

    def _build(self):
        if self._csr is None:
            starts, toks, kids = [0], [], []
            ids = {id(self.trie): 0}
            order = [self.trie]
            i = 0
            while i < len(order):
                node = order[i]
                for t in sorted(node):
                    child = node[t]
                    ids[id(child)] = len(order)
                    order.append(child)
                    toks.append(t)
                    kids.append(ids[id(child)])
                starts.append(len(toks))
                i += 1
            self._csr = (starts, toks, kids)
            self._ids = ids
        return self._csr

    def node_of(self, token_ids) -> int:
        """Node id reached by ``token_ids`` from the root, -1 off the trie."""
        self._build()
        node = self.trie
        for t in token_ids:
            if t not in node:
                return -1
            node = node[t]
        return self._ids[id(node)]

    def to_device(self, device) -> CatalogTensors:
        starts, toks, kids = self._build()
        as_i32 = lambda v: torch.tensor(v, dtype=torch.int32).to(device)
        return CatalogTensors(as_i32(starts), as_i32(toks), as_i32(kids))
