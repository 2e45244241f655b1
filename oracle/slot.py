"""Oracle restatement of the low-entropy-last slot state machine (stream/slot.py:12-176).

Test infrastructure only (see oracle/__init__.py). The random streams are torch's (`randperm` for the block order,
`multinomial` for the categorical draws) on the slot's device, exactly as the reference draws them, so a trajectory
is comparable with the product slot only on the same device and torch build. Selection uses the numpy restatement
in `oracle.sampling` on host copies.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import sampling as S


class ForwardBudget:
    """`ForwardBudget` (stream/slot.py:12-47): one marking forward, then one forward per solid quota."""

    def __init__(self):
        self.phase = 'idle'
        self.solid = 0
        self.left = 0
        self.nfe = 0

    def arm(self, total):
        total = int(total)
        if total < 1:
            raise ValueError('A window needs at least the marking forward')
        self.phase = 'marking'
        self.solid = total - 1
        self.left = 0
        self.nfe = 0

    def forward(self):
        if self.phase == 'idle':
            return False
        self.nfe += 1
        if self.phase == 'marking':
            self.phase = 'solid'
            self.left = self.solid
        else:
            self.left -= 1
        if self.left == 0:
            self.phase = 'idle'
            return True
        return False


class LowEntropyLastSlot:
    """`LowEntropyLastSlot` (stream/slot.py:50-176).

    `air_prob_fn(logits, air_ids)` and `score_fn(logits)` default to the reference torch forms; tests pass the HIP
    values in to check the selection bit for bit given identical scores."""

    def __init__(self, shape, classes, air_ids, air_token, last_eps, block_size, device,
                 score_fn=None, air_prob_fn=None):
        self.shape = tuple(shape)
        self.total = int(np.prod(self.shape))
        self.classes = int(classes)
        self.air_ids = tuple(air_ids)
        self.air_token = int(air_token)
        self.last_eps = float(last_eps)
        self.block_size = int(block_size)
        self.device = torch.device(device)
        self.score_fn = score_fn or (lambda logits: S.entropy_scores(logits.cpu()).numpy())
        self.air_prob_fn = air_prob_fn or (lambda logits, air: S.air_prob(logits.cpu(), air).numpy())
        self.phase = 'idle'
        self.quotas = None
        self.solid_calls = 0
        self.nfe = 0
        self.actual = 0
        self.last_count = 0
        self.step_map = torch.zeros(self.shape, dtype=torch.int16)
        self.values = torch.full(self.shape, -1, dtype=torch.int16)

    @property
    def idle(self):
        return self.phase == 'idle'

    def arm(self, seed, cap, target):
        """stream/slot.py:86-103."""
        self.phase = 'marking'
        self.seed, self.cap, self.target = int(seed), int(cap), tuple(target)
        self.nfe = self.actual = self.solid_calls = self.last_count = 0
        self.quotas = None
        self.last = np.zeros(self.shape, dtype=bool)
        blocks = self.total // self.block_size ** 3
        order_rng = torch.Generator(device=self.device).manual_seed(self.seed + 9173)
        self.order = torch.randperm(blocks, device=self.device, generator=order_rng)
        self.generator = torch.Generator(device=self.device).manual_seed(self.seed)
        self.step_map = torch.zeros(self.shape, dtype=torch.int16)
        self.values = torch.full(self.shape, -1, dtype=torch.int16)

    def time(self):
        """stream/slot.py:110-115."""
        if self.phase == 'idle':
            return 1.0
        committed = sum(self.quotas[:self.solid_calls]) if self.quotas else 0
        return S.actual_time((self.total - committed) / self.total)

    def consume(self, logits, tokens):
        """stream/slot.py:117-164; `tokens` [Y,Z,X] int64 updated in place, `logits` [C,Y,Z,X]."""
        if self.phase == 'idle':
            return None, None
        if self.phase == 'marking':
            self.nfe += 1
            air_p = np.asarray(self.air_prob_fn(logits, self.air_ids), dtype=np.float32)
            ones = np.ones(self.shape, dtype=bool)
            zeros = np.zeros(self.shape, dtype=bool)
            self.last = S.low_entropy_last_update(self.last, ones, air_p, zeros, self.last_eps, False, True)
            self.last_count = int(self.last.sum())
            self.quotas = S.low_entropy_last_quotas(self.total, self.cap, self.last_count, 'quartercos')
            self.phase = 'solid'
            self.solid_calls = 0
            if not self.quotas:
                return self._finish(tokens), None
            return None, None
        if self.solid_calls >= len(self.quotas):
            return self._finish(tokens), None
        k = self.quotas[self.solid_calls]
        tok = tokens.detach().cpu().numpy()
        selectable = (tok == self.classes) & ~self.last
        committed = sum(self.quotas[:self.solid_calls])
        frac = (committed + k) / (self.total - self.last_count)
        n_total = S.block_view(~self.last, self.block_size).sum(1)
        score = np.asarray(self.score_fn(logits), dtype=np.float32)
        chosen = S.block_quota_select(score, selectable, k, self.block_size, self.order.cpu().numpy(), frac, n_total)
        if S.select_bad(chosen, selectable, k):
            raise AssertionError('low-entropy-last solid step did not meet its quota')
        index = torch.from_numpy(np.flatnonzero(chosen)).to(logits.device)
        probabilities = logits.reshape(self.classes, -1).index_select(1, index).t().float().softmax(-1)
        values = torch.multinomial(probabilities, 1, generator=self.generator).squeeze(-1)
        tokens.view(-1).index_copy_(0, index.to(tokens.device), values.to(tokens.device))
        values_cpu = values.to(dtype=torch.int16, device='cpu')
        self.solid_calls += 1
        self.actual += 1
        self.nfe += 1
        positions = index.cpu()
        self.step_map.reshape(-1)[positions] = self.nfe
        self.values.reshape(-1)[positions] = values_cpu
        commit = dict(positions=positions.numpy().astype('int32'), values=values_cpu.numpy(), step=int(self.nfe))
        if self.solid_calls >= len(self.quotas):
            return self._finish(tokens), commit
        return None, commit

    def _finish(self, tokens):
        """stream/slot.py:166-176."""
        last = torch.from_numpy(self.last)
        tokens[last.to(tokens.device)] = self.air_token
        self.step_map[last] = self.nfe
        self.values[last] = self.air_token
        record = dict(target=self.target, seed=self.seed, cap=self.cap, nfe=int(self.nfe), actual=int(self.actual),
                      last_count=int(self.last_count), last_frac=float(self.last_count) / self.total,
                      step_map=self.step_map.clone(), values=self.values.clone())
        self.phase = 'idle'
        self.target = None
        return record
