"""DraftKVPool: the PackedDraft cache state (dspark_qwen/packed_draft.py:63-185)
on a head-major slotted pool.  A host mirror of every request's committed
rows follows random add / append / crop / remove sequences; request_kv must
equal it bit for bit after every step, draft attention over the pool must
pass the oracle gate, and refused appends (nonfinite, capacity, precision)
must leave the pool unchanged."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, randn_bf16
from oracle import cref

pytestmark = pytest.mark.gpu
LAYERS, CAP = 3, 96


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


def new_pool(dev, **kw):
    from qwen3_dspark_amd.draft import DraftKVPool
    args = dict(layers=LAYERS, slots=4, capacity=CAP, device=dev)
    args.update(kw)
    return DraftKVPool(**args)


def projected(gen, rows, form):
    """Per layer (k, v) in the reference's [1, H, rows, D] form or token-major."""
    out = []
    for _ in range(LAYERS):
        k, v = randn_bf16(gen, rows, 8, 128), randn_bf16(gen, rows, 8, 128)
        if form == 'head_major':
            k, v = k.transpose(0, 1)[None].contiguous(), v.transpose(0, 1)[None].contiguous()
        out.append((k, v))
    return out


def token_rows(t):
    """[1, H, n, D] or [n, H, D] -> uint16 [n, H, D]."""
    return bits(t[0].transpose(0, 1)) if t.ndim == 4 else bits(t)


def check_mirror(pool, mirror):
    assert pool.lengths == {r: len(m[0][0]) for r, m in mirror.items()}
    for r, layers in mirror.items():
        kv = pool.request_kv(r)
        for (k, v), (mk, mv) in zip(kv, layers):
            assert k.shape == (1, 8, len(mk), 128)
            assert np.array_equal(token_rows(k), np.asarray(mk, np.uint16).reshape(-1, 8, 128))
            assert np.array_equal(token_rows(v), np.asarray(mv, np.uint16).reshape(-1, 8, 128))


def test_random_append_crop_remove_sequences_bit_exact(dev):
    gen = torch.Generator().manual_seed(SEED)
    rng = np.random.default_rng(7)
    pool = new_pool(dev)
    mirror = {}
    names = iter(f'req{i}' for i in range(100))
    for step in range(40):
        op = rng.choice(['add', 'append', 'append', 'crop', 'remove'])
        if op == 'add' and len(mirror) < 4:
            r = next(names)
            pool.add_request(r)
            mirror[r] = [([], []) for _ in range(LAYERS)]
        elif op == 'append' and mirror:
            chosen = [r for r in mirror if rng.random() < 0.7] or [next(iter(mirror))]
            chunks = {}
            for r in chosen:
                room = CAP - len(mirror[r][0][0])
                if room:
                    chunks[r] = int(rng.integers(1, min(room, 20) + 1))
            if not chunks:
                continue
            form = 'head_major' if rng.random() < 0.5 else 'token_major'
            proj = projected(gen, sum(chunks.values()), form)
            pool.append_projected(chunks, [(k.to(dev), v.to(dev)) for k, v in proj])
            off = 0
            for r, n in chunks.items():
                for l, (k, v) in enumerate(proj):
                    mirror[r][l][0].extend(token_rows(k)[off:off + n].tolist())
                    mirror[r][l][1].extend(token_rows(v)[off:off + n].tolist())
                off += n
        elif op == 'crop' and mirror:
            r = list(mirror)[int(rng.integers(0, len(mirror)))]
            n = int(rng.integers(0, len(mirror[r][0][0]) + 1))
            pool.crop(r, n)
            mirror[r] = [(k[:n], v[:n]) for k, v in mirror[r]]
        elif op == 'remove' and mirror:
            r = list(mirror)[int(rng.integers(0, len(mirror)))]
            pool.remove_request(r)
            del mirror[r]
        check_mirror(pool, mirror)


def test_refused_appends_leave_pool_unchanged(dev):
    gen = torch.Generator().manual_seed(SEED + 1)
    pool = new_pool(dev)
    pool.add_request('a')
    pool.add_request('b')
    base = projected(gen, 10, 'head_major')
    pool.append_projected({'a': 6, 'b': 4}, [(k.to(dev), v.to(dev)) for k, v in base])
    before = [tuple(bits(t) for t in kv) for kv in pool.request_kv('a')]
    bad = projected(gen, 5, 'token_major')
    bad[1][1][2, 3, 7] = float('nan')
    with pytest.raises(RuntimeError, match='Nonfinite'):
        pool.append_projected({'a': 5}, [(k.to(dev), v.to(dev)) for k, v in bad])
    inf = projected(gen, 5, 'token_major')
    inf[2][0][4, 0, 0] = float('inf')
    with pytest.raises(RuntimeError, match='Nonfinite'):
        pool.append_projected({'a': 5}, [(k.to(dev), v.to(dev)) for k, v in inf])
    assert pool.lengths == {'a': 6, 'b': 4}
    after = [tuple(bits(t) for t in kv) for kv in pool.request_kv('a')]
    assert all(np.array_equal(x, y) for p, q in zip(before, after) for x, y in zip(p, q))
    big = projected(gen, CAP, 'token_major')
    with pytest.raises(ValueError, match='capacity'):
        pool.append_projected({'a': CAP}, [(k.to(dev), v.to(dev)) for k, v in big])
    with pytest.raises(ValueError, match='precision'):
        pool.append_projected({'a': 2}, [(k.float().to(dev)[:2], v.float().to(dev)[:2]) for k, v in big])
    with pytest.raises(KeyError):
        pool.append_projected({'zzz': 1}, [(k.to(dev)[:1], v.to(dev)[:1]) for k, v in big])
    with pytest.raises(ValueError, match='crop'):
        pool.crop('a', 7)
    with pytest.raises(ValueError, match='fresh'):
        pool.add_request('a')
    assert pool.lengths == {'a': 6, 'b': 4}


def test_pool_attention_against_oracle(dev):
    gen = torch.Generator().manual_seed(SEED + 2)
    rng = np.random.default_rng(3)
    from qwen3_dspark_amd.draft import DraftKVPool
    pool = DraftKVPool(layers=2, slots=5, capacity=2048, device=dev)
    lengths = {'r0': 700, 'r1': 1500, 'r2': 33, 'r3': 1}
    rows = {}
    for r, n in lengths.items():
        pool.add_request(r)
    # two appends per request, in different chunk orders, so slots fill in place
    for part in (0, 1):
        chunks = {r: (n // 2 if part == 0 else n - n // 2) for r, n in lengths.items()}
        chunks = {r: n for r, n in chunks.items() if n}
        if part:
            chunks = dict(reversed(list(chunks.items())))
        total = sum(chunks.values())
        proj = [(randn_bf16(gen, total, 8, 128), randn_bf16(gen, total, 8, 128)) for _ in range(2)]
        pool.append_projected(chunks, [(k.to(dev), v.to(dev)) for k, v in proj])
        off = 0
        for r, n in chunks.items():
            for l in range(2):
                rows.setdefault((r, l), ([], []))
                rows[(r, l)][0].append(bits(proj[l][0][off:off + n]))
                rows[(r, l)][1].append(bits(proj[l][1][off:off + n]))
            off += n
    pool.crop('r1', 1200)
    lengths['r1'] = 1200
    anchors = {r: [n] + [int(x) for x in rng.integers(0, n + 1, size=int(rng.integers(0, 4)))]
               for r, n in lengths.items()}
    batch = pool.batch(anchors)
    nb = sum(len(a) for a in anchors.values())
    for layer in range(2):
        q, bk, bv = randn_bf16(gen, 7 * nb, 16, 128), randn_bf16(gen, 7 * nb, 8, 128), randn_bf16(gen, 7 * nb, 8, 128)
        out = pool.attention(layer, q.to(dev), bk.to(dev), bv.to(dev), batch)
        ck = np.concatenate([np.concatenate(rows[(r, layer)][0])[:lengths[r]] for r in lengths])
        cv = np.concatenate([np.concatenate(rows[(r, layer)][1])[:lengths[r]] for r in lengths])
        offs = np.concatenate([[0], np.cumsum(list(lengths.values()))[:-1]]).tolist()
        cu_b = np.cumsum([0] + [len(a) for a in anchors.values()])
        ref = cref.draft_attention(bits(q), ck, cv, offs, list(lengths.values()), bits(bk), bits(bv), cu_b,
                                   [x for a in anchors.values() for x in a], scale=SCALE)
        attention_gate(out.float().cpu().numpy(), ref)


def test_more_than_sixteen_layers_append_in_groups(dev):
    """A pool of 20 layers (more than one append launch's 16 pointer slots):
    the append runs per group of 16 layers, and every layer's rows land bit
    for bit, for K and V in one launch and for an fp32-K pool (separate K
    and V launches)."""
    from qwen3_dspark_amd.draft import DraftKVPool
    gen = torch.Generator().manual_seed(SEED + 20)
    for key_dtype, launches in ((torch.bfloat16, 2), (torch.float32, 4)):
        pool = DraftKVPool(layers=20, slots=3, capacity=64, device=dev, key_dtype=key_dtype,
                           value_dtype=torch.bfloat16)
        for r in ('a', 'b'):
            pool.add_request(r)
        rows = {'a': 5, 'b': 9}
        proj = [(randn_bf16(gen, 14, 8, 128).to(key_dtype), randn_bf16(gen, 14, 8, 128)) for _ in range(20)]
        work = pool.append_projected(rows, [(k.to(dev), v.to(dev)) for k, v in proj])
        torch.cuda.synchronize()
        assert work['append_launches'] == launches
        assert pool.lengths == rows
        kv = {r: pool.request_kv(r) for r in rows}
        for layer, (k, v) in enumerate(proj):
            for r, lo, hi in (('a', 0, 5), ('b', 5, 14)):
                gk, gv = kv[r][layer]
                assert torch.equal(gk[0].transpose(0, 1).cpu(), k[lo:hi])
                assert torch.equal(gv[0].transpose(0, 1).cpu(), v[lo:hi])
