"""The per-step records the optimizer hands to the library, built on the host (no GPU needed):
_fill_adam_steps, which writes each run of entries of one group and one step count once and
keeps the hyperparameter columns between calls, gives the same records as filling every field
entry by entry (the form it replaced), over groups, step counts, Magma masks, RAdam, update_rate
and hyperparameters that change between calls."""
import numpy as np
import pytest
import torch

from thorn_amd import _lib
from thorn_amd import optim as O


def _entry_by_entry(entries, update_rate):
    """Every field of every record from its own entry (the per-entry form)."""
    s = np.zeros(len(entries), dtype=_lib.ADAM_TENSOR_STEP)
    steps = [e[1]['step'] for e in entries]
    rect = [O._compute_rect(e[2], st) for e, st in zip(entries, steps)]
    s['p'] = [e[0].data_ptr() for e in entries]
    s['g'] = [e[0].grad.data_ptr() for e in entries]
    s['m'] = [e[1]['moment'].data_ptr() for e in entries]
    s['v'] = [e[1]['variance'].data_ptr() for e in entries]
    s['lr'] = [e[2].lr * r * 1.0 for e, r in zip(entries, rect)]
    s['weight_decay'] = [e[2].weight_decay for e in entries]
    s['beta2'] = [e[2].betas[1] for e in entries]
    s['w1'] = [1 - e[2].betas[0] for e in entries]
    s['w2'] = [1 - e[2].betas[1] for e in entries]
    s['bc1'] = [1 / (1 - e[2].betas[0] ** st) for e, st in zip(entries, steps)]
    s['bc2'] = [1 / (1 - e[2].betas[1] ** st) for e, st in zip(entries, steps)]
    s['eps'] = [e[2].eps for e in entries]
    s['apply'] = [1 if (st + 1) % update_rate == 0 and e[3] else 0 for e, st in zip(entries, steps)]
    s['degenerate'] = [1 if r == 0.0 else 0 for r in rect]
    s['magma_s'] = [e[1]['s'].data_ptr() if e[2].momentum_align else 0 for e in entries]
    return s


def _tensor(n, seed):
    t = torch.randn(n, generator=torch.Generator().manual_seed(seed))
    t.grad = torch.randn(n, generator=torch.Generator().manual_seed(seed + 1000))
    return t


def _group(**kw):
    base = dict(orthogonalize=False, params=[], lr=1e-3, betas=(0.9, 0.95), weight_decay=0.0)
    base.update(kw)
    return O._Group.from_kwargs(**base)


def _state(p, step, magma):
    st = {'step': step, 'moment': torch.zeros_like(p), 'variance': torch.zeros_like(p)}
    if magma:
        st['s'] = torch.ones(())
    return st


@pytest.mark.parametrize('update_rate', [1, 2, 3])
def test_adam_records_equal_entry_by_entry(update_rate):
    ga = _group(lr=1e-3, weight_decay=0.1)
    gb = _group(lr=3e-4, betas=(0.8, 0.99), eps=1e-8, rectify=True)
    gc = _group(lr=2e-3, momentum_align=True)
    ps = [_tensor(5 + i, i) for i in range(9)]
    memo: dict = {}
    s = np.zeros(len(ps), dtype=_lib.ADAM_TENSOR_STEP)
    for step in range(1, 9):
        # group a: one step count; group b: a tensor added later (its own count); group c: Magma
        entries = [(ps[0], _state(ps[0], step, False), ga, True),
                   (ps[1], _state(ps[1], step, False), ga, True),
                   (ps[2], _state(ps[2], step, False), ga, True),
                   (ps[3], _state(ps[3], step, False), gb, True),
                   (ps[4], _state(ps[4], max(1, step - 3), False), gb, True),
                   (ps[5], _state(ps[5], step, False), gb, True),
                   (ps[6], _state(ps[6], step, True), gc, step % 2 == 0),
                   (ps[7], _state(ps[7], step, True), gc, True),
                   (ps[8], _state(ps[8], step, True), gc, step % 3 != 0)]
        if step == 5:   # a scheduler moves the learning rate and the weight decay of group a
            ga = _group(lr=5e-4, weight_decay=0.05)
            entries = [(e[0], e[1], ga if e[2].lr == 1e-3 else e[2], e[3]) for e in entries]
        O._fill_adam_steps(s, entries, update_rate, memo)
        ref = _entry_by_entry(entries, update_rate)
        for name in _lib.ADAM_TENSOR_STEP.names:
            assert np.array_equal(s[name], ref[name]), (step, name, s[name], ref[name])


def test_adam_records_follow_new_run_boundaries():
    """The hyperparameter columns are rewritten when the runs change (an entry moves to another
    group between calls), not only when a value does."""
    ga = _group(lr=1e-3, weight_decay=0.1)
    gb = _group(lr=1e-3, weight_decay=0.2)
    ps = [_tensor(4, 50 + i) for i in range(4)]
    memo: dict = {}
    s = np.zeros(len(ps), dtype=_lib.ADAM_TENSOR_STEP)
    for split in (2, 3, 1, 3):
        entries = [(p, _state(p, 4, False), ga if k < split else gb, True) for k, p in enumerate(ps)]
        O._fill_adam_steps(s, entries, 1, memo)
        ref = _entry_by_entry(entries, 1)
        for name in _lib.ADAM_TENSOR_STEP.names:
            assert np.array_equal(s[name], ref[name]), (split, name)
