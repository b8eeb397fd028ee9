"""Two gfx950 hazards that the compiler does not always see, checked in the library's assembly.

1. A vector memory store of more than 8 bytes reads its data registers after it issues: a VALU
   instruction that writes one of them needs two wait states after the store. The compiler's hazard
   recognizer inserts them, but it counted a scheduling-barrier pseudo-instruction (which emits no
   code) as one; a VALU write right behind a 16-byte store of p then corrupted that store's first
   element, every run a little differently.
2. An LDS DMA load (`buffer_load ... lds`, `global_load_lds_*`) reads M0, and an M0 write needs one
   wait state before it. The library issues these loads from inline assembly, where the compiler's
   recognizer does not look.

The test compiles csrc/thorn_abi.hip to assembly with the library's own flags and walks every
kernel's instruction stream. Wait states: s_nop N counts N + 1, other instructions 1, labels,
directives and comments 0 (a conservative count within a basic block; the scan stops at a label or a
branch).
"""
from __future__ import annotations

import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from thorn_amd import build as B  # noqa: E402

HIPCC = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'

STORE = re.compile(r'\s+(buffer_store_dwordx[34]|buffer_store_b(?:96|128)|global_store_dwordx[34]|'
                   r'global_store_b(?:96|128)|scratch_store_dwordx[34]|scratch_store_b(?:96|128))\s+'
                   r'(v\[\d+:\d+\]|v\d+),\s*(v\[\d+:\d+\]|v\d+)')
VALU_DEF = re.compile(r'\s+(v_\w+)\s+(v\[\d+:\d+\]|v\d+)\b')
NOP = re.compile(r'\s+s_nop\s+(\d+)')
LDS_DMA = re.compile(r'\s+(buffer_load_\w+\s.*\blds\b|global_load_lds_\w+)')
M0_WRITE = re.compile(r'\s+s_\w+\s+m0\b')


def _regs(spec: str) -> set:
    m = re.match(r'v\[(\d+):(\d+)\]', spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r'v(\d+)', spec)
    return {int(m.group(1))} if m else set()


def _is_instr(line: str) -> bool:
    s = line.strip()
    return bool(s) and not s.startswith(';') and not s.startswith('.') and not line.startswith(('.', '_'))


def _wait_states(line: str) -> int:
    m = NOP.match(line)
    return int(m.group(1)) + 1 if m else 1


def _block_end(line: str) -> bool:
    s = line.strip()
    return line.startswith(('.', '_')) or s.startswith(('s_branch', 's_cbranch', 's_setpc', 's_endpgm'))


def store_data_hazards(lines: list) -> list:
    """(line number, store, offending VALU) for every VALU write of a >8-byte store's data register
    with fewer than two wait states after the store."""
    out = []
    for i, line in enumerate(lines):
        m = STORE.match(line)
        if not m:
            continue
        data = _regs(m.group(3)) if m.group(1).startswith(('global', 'scratch')) else _regs(m.group(2))
        waits = 0
        for nxt in lines[i + 1:]:
            if _block_end(nxt) or waits >= 2:
                break
            if not _is_instr(nxt):
                continue
            d = VALU_DEF.match(nxt)
            if d and not d.group(1).startswith(('v_cmp', 'v_readlane', 'v_readfirstlane')) and _regs(d.group(2)) & data:
                out.append((i + 1, line.strip(), nxt.strip()))
                break
            waits += _wait_states(nxt)
    return out


def m0_dma_hazards(lines: list) -> list:
    """(line number, M0 write, LDS DMA) for an LDS DMA load issued right after an M0 write."""
    out = []
    for i, line in enumerate(lines):
        if not M0_WRITE.match(line):
            continue
        for nxt in lines[i + 1:]:
            if _block_end(nxt):
                break
            if not _is_instr(nxt):
                continue
            if LDS_DMA.match(nxt):
                out.append((i + 1, line.strip(), nxt.strip()))
            break
    return out


@pytest.fixture(scope='module')
def asm_lines(tmp_path_factory) -> list:
    if not Path(HIPCC).exists():
        pytest.skip('hipcc not available')
    out = tmp_path_factory.mktemp('isa') / 'thorn_abi.s'
    flags = [f for f in B.HIPCC_FLAGS if f not in ('-shared', '-fPIC')]
    cmd = [HIPCC, *flags, '--offload-device-only', '-S', f'-I{ROOT / "include"}', str(B.SRC), '-o', str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text().split('\n')


def test_store_data_wait_states(asm_lines):
    assert sum(1 for l in asm_lines if STORE.match(l)) > 100   # the scan sees the kernels' stores
    bad = store_data_hazards(asm_lines)
    assert not bad, f'{len(bad)} VALU writes of 16-byte store data within two wait states: {bad[:5]}'


def test_m0_before_lds_dma(asm_lines):
    assert sum(1 for l in asm_lines if LDS_DMA.match(l)) > 50
    bad = m0_dma_hazards(asm_lines)
    assert not bad, f'{len(bad)} LDS DMA loads right after an M0 write: {bad[:5]}'


def test_scanner_flags_the_measured_pattern():
    """The sequence that corrupted p (store, store, scheduling-barrier comment, VALU write of the
    second store's first data register) is flagged; with an s_nop 1 after the stores it is not."""
    bad = ['\tbuffer_store_dwordx4 v[182:185], v208, s[16:19], s25 offen',
           '\tbuffer_store_dwordx4 v[186:189], v208, s[16:19], s25 offen offset:16',
           '\t; sched_barrier mask(0x00000000)',
           '\tv_add_u32_e32 v186, 0x12000, v210']
    assert len(store_data_hazards(bad)) == 1
    good = bad[:2] + ['\ts_nop 1'] + bad[2:]
    assert store_data_hazards(good) == []
    assert len(m0_dma_hazards(['\ts_mov_b32 m0, s81', '\tbuffer_load_dwordx4 v93, s[56:59], 0 offen lds'])) == 1
    assert m0_dma_hazards(['\ts_mov_b32 m0, s81', '\ts_nop 0', '\tbuffer_load_dwordx4 v93, s[56:59], 0 offen lds']) == []
