"""Static check of compiled gfx950 kernels: no barrier inside a divergent loop.

A loop whose latch is exec-masked (s_andn2_b64 exec, exec, ...) lets lanes of
one wave leave it in different iterations. If such a loop contains s_barrier,
part of a wave can arrive at barriers while other lanes of the same wave wait
outside the loop -- the block livelocks or deadlocks even when every value
was uniform at run time. LLVM annotates every basic block with its loop
nesting ("in Loop: Header=BBx Depth=d"); this walks those annotations.
"""
import re


def divergent_barrier_loops(asm_text):
    """Return [(kernel, latch_block, loop_header)] for every violation."""
    out = []
    kernel = None
    blocks = []
    lines = asm_text.split('\n')
    for i, l in enumerate(lines):
        mk = re.match(r'^(_Z\w+):', l)
        if mk:
            out += _check(kernel, blocks)
            kernel, blocks = mk.group(1), []
            continue
        _scan(lines, i, l, blocks)
    out += _check(kernel, blocks)
    return out


def _scan(lines, i, l, blocks):
    m = re.match(r'^(\.LBB(\d+_\d+)|; %bb\.\d+):?', l)
    if m and not l.startswith(';;'):
        cur = {'label': m.group(1), 'inner': None, 'loops': set(), 'lines': []}
        blocks.append(cur)
        ann = [l] + [x for x in lines[i + 1:i + 8] if x.lstrip().startswith(';') and 'Loop' in x]
        best = -1
        for a in ann:
            for h, d in re.findall(r'Header=BB(\d+_\d+) Depth=(\d+)', a):
                cur['loops'].add(h)
                if int(d) > best:
                    best, cur['inner'] = int(d), h
            for h in re.findall(r'Parent Loop BB(\d+_\d+)', a):
                cur['loops'].add(h)
            md = re.search(r'This (?:Inner )?Loop Header: Depth=(\d+)', a)
            if md and m.group(2):
                cur['loops'].add(m.group(2))
                if int(md.group(1)) > best:
                    best, cur['inner'] = int(md.group(1)), m.group(2)
    elif blocks:
        blocks[-1]['lines'].append(l)


def _check(kernel, blocks):
    out = []
    for b in blocks:
        if any('s_andn2_b64 exec, exec' in l for l in b['lines']) and b['inner']:
            h = b['inner']
            body = [x for x in blocks if h in x['loops']]
            if any(any('s_barrier' in l for l in x['lines']) for x in body):
                out.append((kernel, b['label'], 'BB' + h))
    return out


def vm_waits_in_compute_blocks(asm_text, min_math=32):
    """Return [(kernel, block, wait)] for compiler-visible vmcnt waits inside
    basic blocks that carry the k-stage math (>= min_math MFMA/FMA ops).

    The stage loops keep direct-to-LDS loads in flight and wait for the
    stage they are about to compute explicitly, once, right before the stage
    barrier (vmcnt <= LOADS with one barrier per stage, vmcnt = 0 with one
    per pair of stages, when nothing else is in flight); when the whole stage
    is one basic block that wait is in it. Any other vmcnt wait in a compute
    block (after the barrier or after the math has started, or a second one)
    stalls the prefetch on every stage. In a one-wave workgroup the compiler
    drops s_barrier and leaves a "; wave barrier" marker in its place, which
    counts as the barrier here.
    """
    out = []
    kernel, label, lines = None, None, []

    def flush():
        math = sum(1 for l in lines if re.search(r'\bv_(mfma|fmac_f32|fma_f32)', l))
        if math >= min_math:
            pending, accepted, math_seen = None, False, False
            for l in lines:
                if re.search(r'\bv_(mfma|fmac_f32|fma_f32)', l):
                    math_seen = True
                if re.search(r'\bs_barrier\b|; wave barrier', l) and pending and not math_seen:
                    pending, accepted = None, True  # the stage wait
                m = re.search(r's_waitcnt\b.*vmcnt\((\d+)\)', l)
                if m:
                    if pending is None and not accepted and not math_seen:
                        pending = l.strip()
                    else:
                        out.append((kernel, label, l.strip()))
            if pending:
                out.append((kernel, label, pending))

    for l in asm_text.split('\n'):
        mk = re.match(r'^(_Z\w+):', l)
        mb = re.match(r'^(\.LBB\d+_\d+|; %bb\.\d+)', l)
        if mk or mb:
            flush()
            lines = []
            if mk:
                kernel, label = mk.group(1), 'entry'
            else:
                label = mb.group(1)
            continue
        if l.startswith('\t') and (not l.lstrip().startswith(';') or 'wave barrier' in l):
            lines.append(l)
    flush()
    return out
