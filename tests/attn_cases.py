"""Synthetic paged int8 KV caches for the attention tests (CPU oracle pins and
GPU parity).  A case is a set of runs (kernels/attention_ops.mojo:54-91):
run i holds n_i consecutive query tokens at positions base_i, base_i + 1, ...
and owns its own pages, drawn from a shuffled pool of physical pages.

Sliding layers use a ring of `ring_pages` pages per run (page_mask =
ring_pages - 1, as gemma4_topology.mojo:36-40 sets up two pages of
SLIDING_WINDOW rows); full layers use page_mask = -1 and enough pages for
every position of the run."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class AttnCase:
    num_q: int
    num_kv: int
    head_dim: int
    window: int            # 0: full attention
    page_shift: int
    row_mask: int
    page_mask: int
    runs: np.ndarray       # oracle.KV_RUN_DT
    base_rows: np.ndarray  # int32
    q_i8: np.ndarray       # [T, num_q*hd]
    qi_bias: np.ndarray    # [T, num_q]
    f_q: np.ndarray
    k_cache: np.ndarray    # [slots, num_kv*hd]
    k_scale: np.ndarray    # [slots, num_kv]
    v_cache: np.ndarray
    v_scale: np.ndarray
    positions: np.ndarray  # [T] absolute position of each token

    @property
    def T(self):
        return self.q_i8.shape[0]

    def slot(self, tok: int, p: int) -> int:
        """Physical row of position p for token tok's run."""
        r = run_index(self.runs, tok)
        rows = self.base_rows[self.runs[r]["rows_off"]:]
        return int(rows[(p >> self.page_shift) & self.page_mask]) + (p & self.row_mask)

    def kv_range(self, tok: int):
        pos = int(self.positions[tok])
        lo = max(0, pos - self.window + 1) if self.window > 0 else 0
        return lo, pos + 1


def run_index(runs, tok):
    r = 0
    while r + 1 < len(runs) and tok >= runs[r + 1]["buf_start"]:
        r += 1
    return r


def make_case(O, seed, *, num_q, num_kv, head_dim, seqs, page_len, window=0, ring_pages=2,
              spare_pages=3):
    """seqs: [(base_pos, n_tokens), ...], one run each."""
    rng = np.random.default_rng(seed)
    shift = int(np.log2(page_len))
    assert 1 << shift == page_len
    pages_per_run = []
    for base, n in seqs:
        if window > 0:
            pages_per_run.append(ring_pages)
        else:
            pages_per_run.append((base + n + page_len - 1) // page_len)
    total = sum(pages_per_run) + spare_pages
    perm = rng.permutation(total)
    runs, rows, buf, off = [], [], 0, 0
    for (base, n), npg in zip(seqs, pages_per_run):
        runs.append((buf, base, off, npg))
        rows.extend(int(perm[off + j]) * page_len for j in range(npg))
        buf += n
        off += npg
    T = buf
    slots = total * page_len
    kvs = num_kv * head_dim
    k_cache = rng.integers(-127, 128, (slots, kvs), dtype=np.int8)
    v_cache = rng.integers(-127, 128, (slots, kvs), dtype=np.int8)
    k_scale = rng.uniform(1.0, 6.0, (slots, num_kv)).astype(np.float32)
    v_scale = rng.uniform(0.5, 3.0, (slots, num_kv)).astype(np.float32)
    q_i8 = rng.integers(-127, 128, (T, num_q * head_dim), dtype=np.int8)
    f_q = rng.uniform(1.0, 6.0, (T, num_q)).astype(np.float32)
    qi_bias = (q_i8.reshape(T, num_q, head_dim).astype(np.int32).sum(-1) * 128).astype(np.float32)
    positions = np.concatenate([np.arange(b, b + n) for b, n in seqs]).astype(np.int64)
    return AttnCase(num_q, num_kv, head_dim, window, shift, page_len - 1,
                    (ring_pages - 1) if window > 0 else -1, O.kv_runs(runs),
                    np.array(rows, np.int32), q_i8, qi_bias, f_q, k_cache, k_scale, v_cache,
                    v_scale, positions)


def oracle_attention(O, c: AttnCase, s_max=1, with_f32=False):
    return O.flash_attention(c.q_i8, c.qi_bias, c.f_q, c.k_cache, c.k_scale, c.v_cache,
                             c.v_scale, c.runs, c.base_rows, c.num_q, c.num_kv, c.head_dim,
                             c.window, c.page_shift, c.row_mask, c.page_mask, s_max=s_max,
                             with_f32=with_f32)
