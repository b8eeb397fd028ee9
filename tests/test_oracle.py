"""The CPU oracle (oracle/thorn_oracle.py) pinned against the reference's own outputs and closed forms.

Golden vectors come from tests/golden/make_golden.py (the reference itself, run in the build
container). With one CPU thread the restatement reproduces them bit for bit, which also pins the
in-place op order of every step.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import thorn_oracle as O
from tests.golden import workloads

GOLD = Path(__file__).resolve().parent / 'golden'


@pytest.fixture(autouse=True)
def one_thread():
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


def test_coefficients_match_reference():
    z = np.load(GOLD / 'coeffs.npz')
    off = 0
    for k, (l, it, sf, cu) in enumerate(z['settings']):
        it = int(it)
        mine = np.asarray(O.optimal_composition(float(l), it, float(sf), float(cu)))
        np.testing.assert_array_equal(mine, z['coeffs'][off:off + it])
        off += it
        ref_r = [int(x) for x in z['restarts'][k] if x >= 0]
        assert O.gram_ns_restarts(*[tuple(c) for c in mine]) == ref_r


def test_coefficients_closed_form_and_equioscillation():
    # a degenerate interval returns the classic quintic (15/8, -10/8, 3/8)
    a, b, c = O._optimal_quintic(1.0, 1.0)
    assert (a, b, c) == (15 / 8, -10 / 8, 3 / 8)
    # a Remez solution equioscillates: p - 1 reaches +-E at l, the two interior extrema and u
    l, u = 0.1, 1.0
    a, b, c = O._optimal_quintic(l, u)
    xs = np.linspace(l, u, 200001)
    p = a * xs + b * xs ** 3 + c * xs ** 5
    err = np.abs(p - 1)
    E = err.max()
    assert abs(err[0] - E) < 1e-9 and abs(err[-1] - E) < 1e-9
    # a perturbed quintic does worse (optimality)
    p2 = (a * 1.001) * xs + b * xs ** 3 + c * xs ** 5
    assert np.abs(p2 - 1).max() > E


def test_polar_decomp_matches_reference():
    z = np.load(GOLD / 'polar.npz')
    coeffs = tuple(O.optimal_composition(1e-3, 5, 0.03, 0.02))
    restarts = tuple(O.gram_ns_restarts(*coeffs))
    k = 0
    while f'in{k}' in z:
        x = torch.from_numpy(z[f'in{k}'])
        y = O.polar_decomp(x, coeffs, restarts)
        np.testing.assert_array_equal(y.numpy(), z[f'out{k}'])
        k += 1
    assert k == 7


@pytest.mark.parametrize('shape', [(32, 32), (24, 56), (56, 24), (3, 16, 40), (64, 192)])
def test_polar_decomp_closed_form(shape):
    """The f16 iteration equals U phi(S) V^T (f64 SVD) to f16 accuracy, for plain and Gram NS."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(shape, generator=g)
    coeffs = tuple(O.optimal_composition(1e-3, 5, 0.03, 0.02))
    restarts = tuple(O.gram_ns_restarts(*coeffs))
    y = O.polar_decomp(x, coeffs, restarts).double()
    ref = O.polar_closed_form(x, coeffs)
    rel = ((y - ref).norm() / ref.norm()).item()
    assert rel < 1e-2, rel
    # a dropped iteration is caught
    bad = O.polar_closed_form(x, coeffs[:-1])
    assert ((y - bad).norm() / bad.norm()).item() > 3 * rel


def test_pnn_matches_reference_and_invariants():
    z = np.load(GOLD / 'pnn.npz')
    u = torch.from_numpy(z['u_in'].copy())
    p = torch.from_numpy(z['p_in'].copy())
    O.per_neuron_norm_update(p, u, lr=3e-3, weight_decay=0.1)
    np.testing.assert_array_equal(u.numpy(), z['u_out'])
    np.testing.assert_array_equal(p.numpy(), z['p_out'])
    # invariants (without the weight-decay term, which is added to u in place): Frobenius norm
    # kept, row RMS equalized
    u0 = torch.from_numpy(z['u_in']).double()
    u1 = O.per_neuron_norm_update(None, torch.from_numpy(z['u_in'].copy())).double()
    assert abs(u1.norm() / u0.norm() - 1) < 1e-6
    rms = u1.square().mean(dim=-1).sqrt()
    assert (rms.max() / rms.min() - 1) < 1e-5


def test_adam_matches_reference():
    z = np.load(GOLD / 'adam.npz')
    cases = [dict(eps=0.0, weight_decay=0.1, degenerate=False), dict(eps=1e-8, weight_decay=0.0, degenerate=False),
             dict(eps=0.0, weight_decay=0.05, degenerate=True)]
    for k, case in enumerate(cases):
        p = torch.from_numpy(z[f'p{k}'].copy())
        m = torch.from_numpy(z[f'm{k}'].copy())
        v = torch.from_numpy(z[f'v{k}'].copy())
        for step in (1, 2, 7):
            g = torch.from_numpy(z[f'g{k}_{step}'])
            O.adam_update(p, g, m, v, step, beta1=0.9, beta2=0.95, lr=1e-3, **case)
            np.testing.assert_array_equal(p.numpy(), z[f'p{k}_{step}'])
            np.testing.assert_array_equal(m.numpy(), z[f'm{k}_{step}'])
            np.testing.assert_array_equal(v.numpy(), z[f'v{k}_{step}'])


def test_adam_special_case_equals_torch_adam():
    """eps > 0, wd = 0, no rectification: THORN's Adam is torch.optim.Adam's update."""
    g = torch.Generator().manual_seed(3)
    p0 = torch.randn(500, generator=g)
    grads = [torch.randn(500, generator=g) for _ in range(5)]
    p = p0.clone()
    m, v = torch.zeros(500), torch.zeros(500)
    q = torch.nn.Parameter(p0.clone())
    ta = torch.optim.Adam([q], lr=1e-2, betas=(0.9, 0.95), eps=1e-8)
    for s, gr in enumerate(grads, start=1):
        O.adam_update(p, gr, m, v, s, beta1=0.9, beta2=0.95, lr=1e-2, weight_decay=0.0, eps=1e-8)
        q.grad = gr.clone()
        ta.step()
    torch.testing.assert_close(p, q.detach(), rtol=1e-5, atol=1e-7)


def test_rect_equals_radam_term():
    """compute_rect with rectify=True is RAdam's rectification (Liu et al. 2019, eq. in torch.optim.RAdam)."""
    grp = O.Group(orthogonalize=False, params=[], lr=1e-3, rectify=True, betas=(0.9, 0.999))
    b2 = 0.999
    rho_inf = 2 / (1 - b2) - 1
    for t in [1, 2, 5, 6, 10, 100, 1000]:
        rho_t = rho_inf - 2 * t * b2 ** t / (1 - b2 ** t)
        want = ((rho_t - 4) * (rho_t - 2) * rho_inf / ((rho_inf - 4) * (rho_inf - 2) * rho_t)) ** 0.5 if rho_t > 5 else None
        got = O.compute_rect(grp, t)
        if want is not None:
            assert abs(got - want) < 1e-12
        if rho_t <= 4:
            assert got == 0.0
    grp2 = O.Group(orthogonalize=False, params=[], lr=1e-3, rectify=False)
    assert O.compute_rect(grp2, 1) == 1.0   # 0.0 ** 0.0


def test_cautious_weight_decay_closed_form():
    p = torch.tensor([1.0, -1.0, 2.0, -2.0, 0.0])
    u = torch.tensor([0.5, 0.5, -0.5, -0.5, 1.0])
    out = O.cautious_weight_decay(p, u.clone(), 0.1)
    want = torch.tensor([0.5 + 0.1, 0.5, -0.5, -0.5 - 0.2, 1.0])
    torch.testing.assert_close(out, want)


def _run_oracle(build, steps, snap):
    torch.manual_seed(0)
    params, groups, grads = build()
    if isinstance(groups, dict):   # the nn.Module overload
        opt = O.OracleTHORN(groups['module'], **groups['kwargs'])
    else:
        opt = O.OracleTHORN(groups)
    got = {}
    for s in range(1, steps + 1):
        for i, p in enumerate(params):
            p.grad = grads(s, i, p).clone()
        opt.step()
        if s % snap == 0 or s == 1:
            for i, p in enumerate(params):
                got[f's{s}_p{i}'] = p.detach().clone().numpy()
                for k, v in opt.state[p].items():
                    got[f's{s}_{k}{i}'] = v.clone().numpy() if torch.is_tensor(v) else np.asarray(v)
    return got


@pytest.mark.parametrize('name,build,steps,snap', [('traj_config1.npz', workloads.config1, 10, 10),
                                                   ('traj_mixed.npz', workloads.mixed_small, 20, 10),
                                                   ('traj_md.npz', workloads.md_small, 20, 10),
                                                   ('traj_magma.npz', workloads.magma_small, 20, 10),
                                                   ('traj_magma_md.npz', workloads.magma_md_small, 20, 10),
                                                   ('traj_sparse.npz', workloads.sparse_small, 12, 4),
                                                   ('traj_magma_sparse.npz', workloads.magma_sparse_small, 12, 4),
                                                   ('traj_md_adam.npz', workloads.md_adam_small, 20, 10),
                                                   ('traj_md_module.npz', workloads.md_module, 10, 5)])
def test_trajectories_match_reference(name, build, steps, snap):
    z = np.load(GOLD / name)
    got = _run_oracle(build, steps, snap)
    keys = [k for k in z.files if not k.startswith('init_')]
    assert set(keys) == set(got), sorted(set(keys) ^ set(got))
    for k in keys:
        np.testing.assert_array_equal(got[k], z[k], err_msg=k)


def _clone_opt(opt, params_src, params_dst, update_rate):
    """A fresh oracle over params_dst (same groups) carrying opt's state, with update_rate."""
    groups = []
    index = {id(p): i for i, p in enumerate(params_src)}
    for g in opt.param_groups:
        d = {k: v for k, v in g.items() if k != 'params'}
        d['params'] = [params_dst[index[id(p)]] for p in g['params']]
        groups.append(d)
    new = O.OracleTHORN(groups)
    new._update_rate = update_rate
    for ps, pd in zip(params_src, params_dst):
        new.state[pd] = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in opt.state[ps].items()}
    return new


@pytest.mark.parametrize('build,rate', [(workloads.mixed_small, 2), (workloads.mixed_small, 3),
                                        (workloads.md_small, 2)])
def test_update_rate_properties(build, rate):
    """update_rate > 1 (thorn.py:1395, 1483-1486, 1706-1707): the momentum and the Adam moments take
    every gradient; a parameter moves only when its step is due, (step + 1) % rate == 0, and a due
    step is exactly an ordinary step from the same state; on other steps a parameter stays put,
    except that a decouple_md one goes through p / G * softplus(rg) * softplus(cg) with unchanged
    gains."""
    params, groups, grads = build()
    opt = O.OracleTHORN(groups)
    opt._update_rate = rate
    md = {id(p) for g in groups if g.get('decouple_md') for p in g['params']}
    adam = {id(p) for g in groups if not g['orthogonalize'] for p in g['params']}
    beta1 = {id(p): g.get('betas', (0.9, 0.95))[0] for g in groups for p in g['params']}
    for s in range(1, 7):
        due = (s + 1) % rate == 0
        before = [p.detach().clone() for p in params]
        st_before = [{k: (v.clone() if torch.is_tensor(v) else v) for k, v in opt.state[p].items()}
                     for p in params]
        shadow_params = [torch.nn.Parameter(p.detach().clone()) for p in params]
        shadow = _clone_opt(opt, params, shadow_params, 1) if s > 1 else None
        for i, p in enumerate(params):
            p.grad = grads(s, i, p).clone()
            shadow_params[i].grad = grads(s, i, p).clone()
        opt.step()
        if shadow is not None:
            shadow.step()
        for i, p in enumerate(params):
            st = opt.state[p]
            g = grads(s, i, p)
            if id(p) not in md and s > 1:
                m_prev = st_before[i]['moment']
                if id(p) in adam:   # m <- lerp(m, g, 1 - beta1) (thorn.py:876)
                    torch.testing.assert_close(st['moment'], m_prev.lerp(g, 1 - beta1[id(p)]), rtol=0, atol=0)
                else:               # m <- beta1 m + g (thorn.py:1376-1381)
                    torch.testing.assert_close(st['moment'], m_prev * beta1[id(p)] + g, rtol=0, atol=0)
            if due:
                if shadow is not None:   # the same as an ordinary step from the same state
                    assert torch.equal(p.detach(), shadow_params[i].detach()), (s, i)
                    if id(p) not in md and id(p) not in adam:   # (rectified Adam may not move yet)
                        assert not torch.equal(p.detach(), before[i]), (s, i)
            elif id(p) in md and s > 1:
                sb = st_before[i]
                if 'row_gain' in sb:
                    G = torch.nn.functional.softplus(sb['row_gain']) * torch.nn.functional.softplus(sb['col_gain'])
                    want = (before[i] / G) * torch.nn.functional.softplus(sb['row_gain'])
                    want = want * torch.nn.functional.softplus(sb['col_gain'])
                else:
                    G = torch.nn.functional.softplus(sb['gain'])
                    want = (before[i] / G) * G
                assert torch.equal(p.detach(), want), (s, i)
                for k in ('row_gain', 'col_gain', 'gain'):
                    if k in sb:
                        assert torch.equal(st[k], sb[k]), (s, i, k)
            elif id(p) not in md:
                assert torch.equal(p.detach(), before[i]), (s, i)
            assert st['step'] == s + 1


def test_gradient_release_hooks():
    """setup_gradient_release (thorn.py:1755-1776): each backward steps every parameter from its
    hook and drops its gradient; with update_rate = 2 the parameters move on the first backward
    (step 1 is due) and stay put on the second; a second registration without
    ignore_existing_hooks raises."""
    torch.manual_seed(3)
    model = torch.nn.Sequential(torch.nn.Linear(12, 20), torch.nn.Tanh(), torch.nn.Linear(20, 6))
    opt = O.OracleTHORN(model, lr=1e-2, weight_decay=0.1)
    opt.setup_gradient_release(model, update_rate=2)
    x = torch.randn(8, 12)
    for it in range(3):
        before = [p.detach().clone() for p in model.parameters()]
        model(x).square().sum().backward()
        after = list(model.parameters())
        assert all(p.grad is None for p in after)
        moved = [not torch.equal(a.detach(), b) for a, b in zip(after, before)]
        assert all(moved) if it % 2 == 0 else not any(moved), (it, moved)
        assert all(opt.state[p]['step'] == it + 2 for p in after)
    with pytest.raises(ValueError, match='post_accumulate_grad_hooks'):
        O.OracleTHORN(model, lr=1e-2).setup_gradient_release(model)


def _sparse_grad(gen, idx, rows, cols, scale=0.1):
    idx = torch.tensor(idx, dtype=torch.int64)
    vals = torch.randn(len(idx), cols, generator=gen) * scale
    return torch.sparse_coo_tensor(idx[None], vals, (rows, cols))


def test_sparse_adam_matches_torch_sparse_adam():
    """The sparse branch (thorn.py:1667-1700) with eps > 0, no weight decay and no rectification is
    torch.optim.SparseAdam (lazy Adam on the gradient's rows; the two differ only in where eps
    enters the denominator, negligible next to sqrt(v) here); gradients with repeated rows."""
    gen = torch.Generator().manual_seed(21)
    w0 = torch.randn(50, 8, generator=gen)
    w = torch.nn.Parameter(w0.clone())
    ref = torch.nn.Parameter(w0.clone())
    opt = O.OracleTHORN([{'orthogonalize': False, 'params': [w], 'lr': 1e-2, 'betas': (0.9, 0.99),
                          'weight_decay': 0.0, 'eps': 1e-8}])
    tref = torch.optim.SparseAdam([ref], lr=1e-2, betas=(0.9, 0.99), eps=1e-8)
    for idx in ([3, 7, 3, 12], [0, 49, 7], [3, 3, 3], [10, 11, 12, 13, 14, 7]):
        g = _sparse_grad(gen, idx, 50, 8)
        w.grad = g.clone()
        ref.grad = g.clone()
        opt.step()
        tref.step()
        torch.testing.assert_close(w.detach(), ref.detach(), rtol=1e-5, atol=1e-7)
        torch.testing.assert_close(opt.state[w]['moment'], tref.state[ref]['exp_avg'], rtol=1e-6, atol=1e-9)
        torch.testing.assert_close(opt.state[w]['variance'], tref.state[ref]['exp_avg_sq'], rtol=1e-6, atol=1e-12)


def test_sparse_rows_invariants():
    """Rows outside the gradient keep parameter and state bit for bit; repeated rows act as their
    sum (coalesce); an empty gradient takes no step at all (thorn.py:1677-1678); a gradient that
    is not row-sparse (sparse_dim 2) becomes dense and takes the dense step."""
    gen = torch.Generator().manual_seed(5)
    grp = {'orthogonalize': False, 'lr': 1e-2, 'betas': (0.9, 0.95), 'weight_decay': 0.1}
    w0 = torch.randn(20, 6, generator=gen)
    a, b, c = (torch.nn.Parameter(w0.clone()) for _ in range(3))
    oa = O.OracleTHORN([dict(grp, params=[a])])
    ob = O.OracleTHORN([dict(grp, params=[b])])
    oc = O.OracleTHORN([dict(grp, params=[c])])
    for s in range(3):
        vals = torch.randn(3, 6, generator=gen) * 0.1
        a.grad = torch.sparse_coo_tensor(torch.tensor([[4, 9, 4]]), vals, (20, 6))
        b.grad = torch.sparse_coo_tensor(torch.tensor([[4, 9]]), torch.stack([vals[0] + vals[2], vals[1]]), (20, 6))
        dense = torch.zeros(20, 6)
        dense[4] = vals[0] + vals[2]
        dense[9] = vals[1]
        c.grad = dense.to_sparse(2)
        before = a.detach().clone()
        oa.step()
        ob.step()
        oc.step()
        assert torch.equal(a.detach(), b.detach())
        keep = [i for i in range(20) if i not in (4, 9)]
        assert torch.equal(a.detach()[keep], before[keep])
        assert not torch.equal(a.detach()[[4, 9]], before[[4, 9]])
        for k in ('moment', 'variance'):
            assert torch.equal(oa.state[a][k][keep], torch.zeros(len(keep), 6))
    # the dense (sparse_dim 2) one takes the dense step: weight decay reaches the untouched rows
    # (u = 0 there passes the cautious mask), which the row-sparse step leaves alone
    assert not torch.equal(c.detach()[keep], a.detach()[keep])
    assert c.grad is None
    step = oa.state[a]['step']
    before = a.detach().clone()
    a.grad = torch.sparse_coo_tensor(torch.zeros(1, 0, dtype=torch.int64), torch.zeros(0, 6), (20, 6))
    oa.step()
    assert oa.state[a]['step'] == step and a.grad is not None and torch.equal(a.detach(), before)


def test_w1rand_matches_reference():
    """Magma's PRNG (thorn.py:800-804) against the reference's own sequences, 40 draws per seed."""
    z = np.load(GOLD / 'magma.npz')
    for seed, states, draws in zip(z['w1_seeds'], z['w1_states'], z['w1_draws']):
        st = int(seed)
        for want_s, want_d in zip(states, draws):
            st, d = O.w1rand(st)
            assert (st, d) == (int(want_s), int(want_d))
    assert {int(d) & 1 for d in z['w1_draws'].ravel()} == {0, 1}


def test_momentum_aligned_mask_matches_reference():
    """_momentum_aligned_mask (thorn.py:806-836): the scale it returns, the new s and the new PRNG
    state, for a zero moment, aligned, opposed and random moments, an explicit `moment` (the
    sparse path's gathered rows) and a moment too small to normalize."""
    z = np.load(GOLD / 'magma.npz')
    grp = O.Group(orthogonalize=False, params=[], lr=1e-3, momentum_align=True)
    scales = []
    for k in range(int(z['n_mask'])):
        g, m = torch.from_numpy(z[f'mask{k}_g']), torch.from_numpy(z[f'mask{k}_m'])
        state = {'s': torch.tensor(float(z[f'mask{k}_s0'])), 'random_state': int(z[f'mask{k}_seed'])}
        if bool(z[f'mask{k}_rows']):
            state['moment'] = torch.full_like(m, 123.0)
            scale = O.momentum_aligned_mask(g, state, grp, moment=m)
        else:
            state['moment'] = m
            scale = O.momentum_aligned_mask(g, state, grp)
        assert scale == float(z[f'mask{k}_scale']), k
        np.testing.assert_array_equal(state['s'].numpy(), z[f'mask{k}_s1'], err_msg=str(k))
        assert state['random_state'] == int(z[f'mask{k}_state1'])
        scales.append(scale)
    assert 0.0 in scales and any(s > 0 for s in scales)


def test_momentum_aligned_mask_closed_forms():
    """s_t = sigmoid(cos / 2) with the pre-update moment: exactly aligned, opposed and orthogonal
    moments give sigmoid(1/2), sigmoid(-1/2) and 1/2; a zero moment gives 1/2 (the norms are
    clamped at 1e-8); an odd PRNG draw returns 0.0 and still moves s and the PRNG state."""
    grp = O.Group(orthogonalize=False, params=[], lr=1e-3, momentum_align=True)
    g = torch.tensor([3.0, -4.0, 0.0, 12.0])
    even = next(s for s in range(100) if O.w1rand(s)[1] % 2 == 0)
    odd = next(s for s in range(100) if O.w1rand(s)[1] % 2 == 1)
    for m, want in [(2.5 * g, 1 / (1 + math.exp(-0.5))), (-0.1 * g, 1 / (1 + math.exp(0.5))),
                    (torch.tensor([4.0, 3.0, 7.0, 0.0]), 0.5), (torch.zeros(4), 0.5)]:
        state = {'s': torch.tensor(1.0), 'moment': m, 'random_state': even}
        scale = O.momentum_aligned_mask(g, state, grp)
        assert abs(state['s'].item() - (0.9 + 0.1 * want)) < 1e-6
        assert scale == state['s'].item()
        assert state['random_state'] == O.w1rand(even)[0]
        state = {'s': torch.tensor(0.5), 'moment': m, 'random_state': odd}
        assert O.momentum_aligned_mask(g, state, grp) == 0.0
        assert abs(state['s'].item() - (0.45 + 0.1 * want)) < 1e-6
