"""Host-side API parity with the reference (CPU only): constructor, groups, defaults, errors."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

import thorn_amd
from oracle import thorn_oracle as O


class Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed = nn.Embedding(10, 4)
        self.proj = nn.Linear(4, 6)
        self.conv = nn.Conv1d(2, 3, 5)
        self.lm_head = nn.Linear(6, 10, bias=False)
        self.norm = nn.LayerNorm(6)


def test_auto_assign_matches_reference_rules():
    m = Tiny()
    opt = thorn_amd.THORN(m, lr=1e-3)
    ref = O.OracleTHORN(m, lr=1e-3)
    ids = lambda groups: [[id(p) for p in g['params']] for g in groups]
    assert ids(opt.param_groups) == ids(ref.param_groups)
    ortho = {id(p) for p in opt.param_groups[0]['params']}
    assert id(m.proj.weight) in ortho and id(m.conv.weight) in ortho
    assert id(m.embed.weight) not in ortho and id(m.lm_head.weight) not in ortho


def test_group_defaults_match_reference():
    p = nn.Parameter(torch.zeros(3, 3))
    opt = thorn_amd.THORN([{'orthogonalize': True, 'params': [p], 'lr': 1e-3}])
    ref = O.OracleTHORN([{'orthogonalize': True, 'params': [nn.Parameter(torch.zeros(3, 3))], 'lr': 1e-3}])
    a = {k: v for k, v in opt.param_groups[0].items() if k != 'params'}
    b = {k: v for k, v in ref.param_groups[0].items() if k != 'params'}
    assert a == b
    assert list(a) == list(b)


def test_ortho_group_rejects_vectors():
    with pytest.raises(AssertionError, match='ndim >= 2'):
        thorn_amd.THORN([{'orthogonalize': True, 'params': [nn.Parameter(torch.zeros(3))], 'lr': 1e-3}])


@pytest.mark.parametrize('bad,msg', [({'lr': -1.0}, 'learning rate'), ({'betas': (1.0, 0.9)}, 'beta1'),
                                     ({'betas': (0.9, 1.5)}, 'beta2')])
def test_invalid_hyperparameters_raise_value_error_at_step(bad, msg):
    p = nn.Parameter(torch.zeros(3, 3))
    opt = thorn_amd.THORN([{'orthogonalize': True, 'params': [p], 'lr': 1e-3, **bad}])
    p.grad = torch.zeros(3, 3)
    with pytest.raises(ValueError, match=msg):
        opt.step()


def test_unsupported_features_raise_not_implemented():
    """decouple_md runs on Adam groups too; a norm axis across the leading dims (not the trailing
    matrix, its rows or its columns) is refused before anything is computed."""
    p = nn.Parameter(torch.zeros(2, 3, 3))
    opt = thorn_amd.THORN([{'orthogonalize': False, 'params': [p], 'lr': 1e-3, 'decouple_md': True,
                            'norm_axis': 0}])
    p.grad = torch.zeros(2, 3, 3)
    with pytest.raises(NotImplementedError, match='norm_axis=0'):
        opt.step()


def test_cpu_tensors_are_refused_not_computed():
    p = nn.Parameter(torch.zeros(3, 3))
    opt = thorn_amd.THORN([{'orthogonalize': True, 'params': [p], 'lr': 1e-3}])
    p.grad = torch.ones(3, 3)
    with pytest.raises(RuntimeError, match='device tensors'):
        opt.step()
    assert torch.count_nonzero(p) == 0


def test_coefficients_match_reference_goldens_exactly():
    """The product's host solver reproduces the reference's coefficient tables bit for bit."""
    from pathlib import Path
    import numpy as np
    from thorn_amd import _coeffs
    z = np.load(Path(__file__).resolve().parent / 'golden' / 'coeffs.npz')
    off = 0
    for k, (l, it, sf, cu) in enumerate(z['settings']):
        it = int(it)
        a = np.asarray(_coeffs.ns_coefficients(float(l), it, float(sf), float(cu)))
        np.testing.assert_array_equal(a, z['coeffs'][off:off + it])
        off += it
        assert list(_coeffs.gram_restarts(tuple(map(tuple, a)))) == [int(x) for x in z['restarts'][k] if x >= 0]


def test_reference_import_path():
    """``from thorn import THORN`` (the reference's thorn/__init__.py:1) gives this build's class."""
    import thorn
    from thorn import THORN
    assert THORN is thorn_amd.THORN
    assert thorn.__all__ == ['THORN', 'THORNOrthoGroup', 'THORNNonOrthoGroup', 'THORNGroup']
    assert thorn.THORNOrthoGroup is thorn_amd.THORNOrthoGroup


def test_polar_decomp_batches():
    """polar_decomp_batch_size (thorn.py:1237, 1440): consecutive parameters, at most the limit's
    elements per batch, a larger parameter alone, and 0 = every parameter alone."""
    from thorn_amd.optim import _batches
    ps = [torch.zeros(n) for n in (5, 3, 4, 10, 1, 1)]
    sizes = lambda bs: [[p.numel() for p in b] for b in bs]
    assert sizes(_batches(ps, 8)) == [[5, 3], [4], [10], [1, 1]]
    assert sizes(_batches(ps, 0)) == [[5], [3], [4], [10], [1], [1]]
    assert sizes(_batches(ps, 1 << 31)) == [[5, 3, 4, 10, 1, 1]]
    assert thorn_amd.THORN.polar_decomp_batch_size == 2 * 1024 ** 3


def test_unsupported_dtypes_are_refused():
    """fp32, bf16, fp16 and fp64 parameters step (the last three through fp32 working copies);
    other dtypes (complex, fp8) raise before anything is computed."""
    from thorn_amd import optim as OPT
    assert set(OPT._DTYPES) == {torch.float32, torch.bfloat16, torch.float16, torch.float64}
    for dt in (torch.complex64, torch.float8_e4m3fn):
        p = nn.Parameter(torch.zeros(3, 3, dtype=dt), requires_grad=False)
        opt = thorn_amd.THORN([{'orthogonalize': True, 'params': [p], 'lr': 1e-3}])
        p.grad = torch.zeros(3, 3, dtype=dt)
        with pytest.raises(NotImplementedError, match='fp32, bf16, fp16 and fp64'):
            opt.step()


def test_chain_split_and_count():
    """The chained group step deals a group's matrices to chains: every parameter exactly once,
    each chain in the group's order, costs (s^2 * l) balanced by the snake deal; two chains up to
    CHAIN_MAX_COST of work (Qwen3-300M set), one plan above (Qwen3-1.7B set). The split itself is
    checked for 2, 3 and 4 chains."""
    import bench
    from thorn_amd import optim as OPT
    for config, want in ((2, 2), (5, 1)):
        mats, _ = bench.config_shapes(config)
        assert OPT._chain_count([torch.empty(sh, device='meta') for sh in mats]) == want
    for config, n in ((2, 2), (5, 2), (5, 3), (5, 4)):
        mats, _ = bench.config_shapes(config)
        params = [torch.empty(sh, device='meta') for sh in mats]
        chains = OPT._split_chains(params, n)
        ids = [id(p) for c in chains for p in c]
        assert sorted(ids) == sorted(id(p) for p in params)
        order = {id(p): i for i, p in enumerate(params)}
        for c in chains:
            pos = [order[id(p)] for p in c]
            assert pos == sorted(pos)
        costs = [sum(OPT._ns_cost(p) for p in c) for c in chains]
        assert max(costs) - min(costs) <= max(OPT._ns_cost(p) for p in params)
    params = [torch.empty(1024, 384, device='meta')] * 3
    assert OPT._chain_count(params) == 2
    assert [len(c) for c in OPT._split_chains(params, 2)] == [1, 2]   # A B B


def test_runner_cache_keeps_one_runner_per_parameter():
    """Gradient release steps each parameter on its own: its runners (one per parameter) are kept,
    up to the group's parameter count, apart from the runners of parameter subsets, of which the
    two most recently used are kept."""
    ps = [nn.Parameter(torch.zeros(4, 4)) for _ in range(3)]
    opt = thorn_amd.THORN([{'params': ps, 'orthogonalize': True}])
    built = []

    def get(ids):
        key = ('ortho', 0, 'dev', tuple(ids), ())
        return opt._runner(key, lambda: built.append(ids) or object())

    for _ in range(3):                       # three steps of gradient release: built once each
        for i in range(3):
            get([i])
    assert built == [[0], [1], [2]]
    get([0, 1]); get([1, 2]); get([0, 2])   # subsets: the two most recent are kept
    keys = [k[3] for k in opt._runners]
    assert (0, 1) not in keys and (1, 2) in keys and (0, 2) in keys
    assert all((i,) in keys for i in range(3))
    get([3])                                 # a fourth single-parameter key evicts the oldest one
    assert sum(1 for k in opt._runners if len(k[3]) == 1) == 3


def test_runner_cache_keeps_gradient_release_windows():
    """Gradient release steps windows of parameters (RELEASE_WINDOW_BYTES of gradients each): their
    runners are kept apart, up to the group's parameter count, whatever the windows' sizes, and do
    not displace the runners of the group's own steps."""
    from thorn_amd import optim as OPT
    ps = [nn.Parameter(torch.zeros(4, 4)) for _ in range(4)]
    opt = thorn_amd.THORN([{'params': ps, 'orthogonalize': True}])
    built = []

    def get(kind, ids):
        return opt._runner((kind, 0, 'dev', tuple(ids), ()), lambda: built.append((kind, ids)) or object())

    get('ortho', [0, 1, 2, 3])
    for _ in range(3):                       # three backward passes with the same windows
        get('release', [3, 2]); get('release', [1]); get('release', [0])
    assert built == [('ortho', [0, 1, 2, 3]), ('release', [3, 2]), ('release', [1]), ('release', [0])]
    get('release', [3]); get('release', [2, 1, 0])   # other windows: the oldest ones go beyond 4
    kinds = [(k[0], k[3]) for k in opt._runners]
    assert ('ortho', (0, 1, 2, 3)) in kinds and ('release', (3, 2)) not in kinds
    assert sum(1 for k in kinds if k[0] == 'release') == 4
    assert OPT._window_full(OPT.RELEASE_WINDOW_BYTES) and not OPT._window_full(OPT.RELEASE_WINDOW_BYTES - 1)


def test_gradient_release_on_cpu_steps_at_once():
    """Parameters off the GPU (and small or non-orthogonalized ones) never wait in a window: the
    hook's step runs at once."""
    p = nn.Parameter(torch.zeros(4, 4))
    opt = thorn_amd.THORN([{'params': [p], 'orthogonalize': True}])
    p.grad = torch.ones(4, 4)
    called = []
    opt.step = lambda closure=None, *, param=None: called.append(param)
    opt._release_step(p, join_later=True)
    assert called == [p] and not opt._release_windows


def test_adam_beside_chains_decision():
    """step() runs the non-orthogonalized groups on a side stream only beside an orthogonalized group
    that steps as chains (config 2: yes; config 5, one plan: no), with dense
    gradients, and when the batch limit keeps the matrices one plan."""
    import bench
    from thorn_amd import optim as OPT

    def params(shapes):
        ps = [nn.Parameter(torch.empty(sh, device='meta')) for sh in shapes]
        for p in ps:
            p.grad = torch.empty(p.shape, device='meta')
        return ps

    emb = nn.Parameter(torch.zeros(10, 4))   # a row-sparse embedding gradient
    emb.grad = torch.sparse_coo_tensor(torch.tensor([[1, 3]]), torch.ones(2, 4), (10, 4))

    m2, o2 = bench.config_shapes(2)
    m5, _ = bench.config_shapes(5)
    adam = [sh for shapes, _ in o2 for sh in shapes]
    big = 2 * 1024 ** 3
    assert OPT._adam_beside_chains([(True, params(m2)), (False, params(adam))], big, {})
    assert OPT._adam_beside_chains([(False, params(adam)), (True, params(m2))], big, {})
    assert not OPT._adam_beside_chains([(True, params(m5)), (False, params(adam))], big, {})      # one plan
    assert not OPT._adam_beside_chains([(True, params(m2[:15])), (False, params(adam))], big, {})  # no chains
    assert not OPT._adam_beside_chains([(True, params(m2)), (False, params(adam) + [emb])], big, {})
    assert not OPT._adam_beside_chains([(True, params(m2)), (False, [])], big, {})
    assert not OPT._adam_beside_chains([(True, params(m2)), (False, params(adam))], 1 << 24, {})  # batches
    cache = {}
    ps = params(m2)
    OPT._adam_beside_chains([(True, ps), (False, params(adam))], big, cache)
    assert list(cache.values()) == [True] and list(cache)[0][0] == tuple(id(p) for p in ps)
    # one 3-D parameter of 28 large matrices is one plan, never chains: no side stream either
    stacked = params([(28, 1024, 1024)])
    assert OPT._large_matrices(stacked) == 28
    assert OPT._chain_plan(stacked, big) is None
    assert not OPT._adam_beside_chains([(True, stacked), (False, params(adam))], big, {})
    # the decision is the chained step's own: _chain_plan on the same parameters
    for shapes, want in ((m2, 2), (m5, None), (m2[:15], None)):
        ch = OPT._chain_plan(params(shapes), big)
        assert (None if ch is None else len(ch)) == want


def test_status_watch_raises_for_a_set_status_word():
    """The small-matrix launch's status word, read into a ring of pinned slots: a completed slot
    holding a nonzero word raises RuntimeError at the next check (not before its event completes,
    unless the check waits), once, and clears the word on the device; reads happen every PERIOD
    steps that ran the launch."""
    from thorn_amd import optim as OPT

    class Ev:
        def __init__(self):
            self.done = False
            self.waited = 0

        def query(self):
            return self.done

        def synchronize(self):
            self.waited += 1
            self.done = True

    class Runner:
        workspace = torch.zeros(1024, dtype=torch.uint8)

    w = OPT._StatusWatch.__new__(OPT._StatusWatch)
    w.runner = Runner()
    w.host = torch.zeros(w.SLOTS, dtype=torch.int32)
    w.events = [Ev() for _ in range(w.SLOTS)]
    w.pending = [False] * w.SLOTS
    w.next = 0
    w.unread = 0
    w.stream = None
    Runner.workspace[256:260].view(torch.int32).fill_(1)   # the device word, set by a timeout
    # slots 0 and 1 recorded; slot 1's step timed out and has not completed yet
    w.pending[0] = w.pending[1] = True
    w.next = 2
    w.host[1] = 1
    w.events[0].done = True
    w.check()                        # slot 0 completed clean; slot 1 still in flight
    assert w.pending == [False, True, False, False] and w.events[1].waited == 0
    with pytest.raises(RuntimeError, match='timed out'):
        w.check(wait=True)
    assert w.pending == [False] * w.SLOTS and int(w.host[1]) == 0
    assert int(Runner.workspace[256:260].view(torch.int32)) == 0   # cleared
    w.check(wait=True)               # reported once
    # reads every PERIOD steps
    reads = []
    w.record = lambda: reads.append(w.unread) or setattr(w, 'unread', 0)
    for _ in range(2 * w.PERIOD + 3):
        w.stepped(None)
    assert reads == [w.PERIOD, w.PERIOD] and w.unread == 3
    # a clean word never raises, completed or waited for
    w.pending[3] = True
    w.events[3].done = True
    w.check()
    assert not any(w.pending)



def test_sym_addmm_op_registration_and_checks():
    """thorn::sym_addmm is registered as in the reference (thorn.py:298): the fake impl gives the
    (..., M, M) result shape on meta tensors, the reference's argument checks raise AssertionError,
    and tensors the library does not take (CPU, float32) are refused rather than computed."""
    import thorn_amd  # noqa: F401  (registers the op)
    op = torch.ops.thorn.sym_addmm
    A = torch.empty(2, 3, 40, 70, device='meta', dtype=torch.float16)
    B = torch.empty(2, 3, 70, 40, device='meta', dtype=torch.float16)
    assert op(A, B, None, 1.0, 1.0).shape == (2, 3, 40, 40)
    assert op(A, B, torch.empty(40, 40, device='meta', dtype=torch.float16), 2.0, 0.5).shape == (2, 3, 40, 40)
    # the checks run before anything is computed (the fake impl, like the reference's, has none)
    a, b = torch.zeros(2, 3, 40, 70, dtype=torch.float16), torch.zeros(2, 3, 70, 40, dtype=torch.float16)
    with pytest.raises(AssertionError, match='B must be'):
        op(a, a, None, 1.0, 1.0)
    with pytest.raises(AssertionError, match='C must be'):
        op(a, b, torch.zeros(2, 40, 41, dtype=torch.float16), 1.0, 1.0)
    with pytest.raises(AssertionError, match='C must be'):
        op(a, b, torch.zeros(3, 40, 40, dtype=torch.float16), 1.0, 1.0)
    with pytest.raises(NotImplementedError, match='float16 CUDA'):
        op(torch.zeros(4, 6, dtype=torch.float16), torch.zeros(6, 4, dtype=torch.float16), None, 1.0, 1.0)
