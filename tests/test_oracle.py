"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against the reference's own known answers,
a library routine or a closed form, chosen so that a plausible mistake (a
transposed pair convention, a dropped scale, a wrong head map, a wrong mask
column order) fails at least one test.  ``test_planted_mistakes_are_caught``
plants such mistakes in copies of the oracle and checks the pins catch them.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kvattn_oracle as orc

GOLD = Path(__file__).resolve().parent / "golden"


def golden():
    return json.loads((GOLD / "golden.json").read_text())


# ---------------------------------------------------------------- RoPE tables
def test_rope_fixture_matches_restatement():
    fx = np.load(GOLD / "rope_0_255.npz")
    cos, sin = orc.rope_tables(256)
    assert cos.dtype == np.float16 and cos.shape == (256, 32)
    assert np.array_equal(cos.view(np.uint16), fx["cos"].view(np.uint16))
    assert np.array_equal(sin.view(np.uint16), fx["sin"].view(np.uint16))


def test_rope_table_hash_full_range():
    from mi50grad_amd.rope import table_digest

    g = golden()
    cos, sin = orc.rope_tables(g["rope_rows"])
    assert table_digest(cos, sin) == g["rope_sha256"], (
        f"RoPE table bits differ from the fixture made with numpy {g['numpy_version']} "
        f"(this numpy: {np.__version__})")


def test_product_rope_table_hash_full_range():
    """The tables the product uploads (mi50grad_amd.rope.rope_tables, used by
    attention._init_rope_tables and the GPU tests' cos/sin) are pinned to the
    same golden digest over rows 0..32776, the positions configs 3 and 5
    reach, not only through the oracle's restatement."""
    from mi50grad_amd.rope import rope_tables, table_digest

    g = golden()
    cos, sin = rope_tables(g["rope_rows"])
    assert cos.shape == (g["rope_rows"], 32)
    assert table_digest(cos, sin) == g["rope_sha256"]


def test_rope_table_closed_form():
    cos, sin = orc.rope_tables(4096)
    # Position 0 is the identity rotation.
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    # Frequency i is theta^(-2i/64); compare with float64 within fp16 rounding
    # plus the float32 angle error (|angle| <= 4096 rad -> ~2.4e-4 abs).
    i = np.arange(32)
    ang = np.arange(4096)[:, None] * 1e7 ** (-2.0 * i / 64.0)
    tol = 2.0 ** -11 + 4096 * 2.0 ** -24 * 2
    assert np.max(np.abs(cos.astype(np.float64) - np.cos(ang))) <= tol
    assert np.max(np.abs(sin.astype(np.float64) - np.sin(ang))) <= tol
    # Frequency 0 is 1 rad per position: sin(1) in fp16.
    assert sin[1, 0] == np.float16(np.sin(1.0))


# ------------------------------------------------------- QK-norm + RoPE (a2/a3)
def _norm_rope_f64(x, w, c, s, eps=1e-6):
    """Textbook float64: RMSNorm with weight, then complex rotation of pairs."""
    x = x.astype(np.float64)
    n = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w.astype(np.float64)
    half = c.shape[-1]
    z = n[:, 0:2 * half:2] + 1j * n[:, 1:2 * half:2]
    z = z * (c.astype(np.float64) + 1j * s.astype(np.float64))
    out = n.copy()
    out[:, 0:2 * half:2] = z.real
    out[:, 1:2 * half:2] = z.imag
    return out


@pytest.mark.parametrize("head_dim,half", [(256, 32), (128, 32), (64, 16)])
def test_qknorm_exact_vs_float64(head_dim, half):
    rng = np.random.default_rng(3)
    n = 40
    x = (rng.standard_normal((n, head_dim)) * 2).astype(np.float16)
    w = (1 + 0.02 * rng.standard_normal(head_dim)).astype(np.float16)
    pos = rng.integers(0, 30000, n)
    cos, sin = orc.rope_tables(30000, head_dim=head_dim, partial_rotary_factor=2 * half / head_dim)
    got = orc.qknorm_rope_exact(x, w, cos[pos], sin[pos]).astype(np.float64)
    ref = _norm_rope_f64(x, w, cos[pos].astype(np.float64), sin[pos].astype(np.float64))
    # Within one fp16 ulp of the exact value (plus fp32 noise).
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp * 1.01 + 1e-7)


def test_qknorm_exact_vs_reference_test_recipe():
    """tests/test_qknorm_rope.py:55-114: seed 42, x*0.3, w in [0.5,1],
    cos/sin(i*0.1), tolerance 2e-3, heads {8, 1, 48} x head_dim {256, 128}."""
    for heads, hd in [(8, 256), (1, 256), (48, 256), (8, 128)]:
        np.random.seed(42)
        x = (np.random.randn(heads, hd) * 0.3).astype(np.float16)
        w = (np.random.rand(hd) * 0.5 + 0.5).astype(np.float16)
        c = np.cos(np.arange(32, dtype=np.float32) * 0.1).astype(np.float16)
        s = np.sin(np.arange(32, dtype=np.float32) * 0.1).astype(np.float16)
        ref = orc.qknorm_rope_float(x, w, np.tile(c, (heads, 1)), np.tile(s, (heads, 1)))
        got = orc.qknorm_rope_exact(x, w, np.tile(c, (heads, 1)), np.tile(s, (heads, 1)))
        assert np.max(np.abs(got.astype(np.float32) - ref.astype(np.float32))) < 2e-3


def test_qknorm_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 256)).astype(np.float16)
    w = (1 + 0.02 * rng.standard_normal(256)).astype(np.float16)
    cos, sin = orc.rope_tables(5000)
    pos = rng.integers(1, 5000, 16)
    rot = orc.qknorm_rope_exact(x, w, cos[pos], sin[pos])
    ident = orc.qknorm_rope_exact(x, w, cos[np.zeros(16, int)], sin[np.zeros(16, int)])
    # Tail dims 64.. carry the norm only, independent of the position.
    assert np.array_equal(rot[:, 64:].view(np.uint16), ident[:, 64:].view(np.uint16))
    # Position 0 (cos=1, sin=0) leaves the normalised values unrotated:
    # the result equals the float64 norm rounded to fp16 within 1 ulp.
    nrm = _norm_rope_f64(x, w, np.ones((16, 32)), np.zeros((16, 32)))
    assert np.all(np.abs(ident.astype(np.float64) - nrm) <= np.spacing(np.abs(nrm).astype(np.float16)))
    # Rotation preserves each pair's norm (to fp16 rounding).
    a = rot[:, 0:64].astype(np.float64).reshape(16, 32, 2)
    b = ident[:, 0:64].astype(np.float64).reshape(16, 32, 2)
    ra, rb = np.linalg.norm(a, axis=-1), np.linalg.norm(b, axis=-1)
    assert np.max(np.abs(ra - rb) / np.maximum(rb, 1e-3)) < 3e-3


def test_qknorm_golden_c1():
    fx = np.load(GOLD / "c1_golden.npz")
    cos, sin = orc.rope_tables(256)
    qn = orc.qknorm_rope_exact(fx["q"][0], fx["q_norm"], np.repeat(cos[255:256], 24, 0),
                               np.repeat(sin[255:256], 24, 0))
    assert np.array_equal(qn.view(np.uint16), fx["q_normed"].view(np.uint16))


# ------------------------------------------------------------- attention (a6-a9)
def _sdpa64(q, k, v, vis=None):
    """torch's scaled_dot_product_attention in float64 on the CPU, GQA by
    repeating each KV head for its group (head h -> kv head h // G)."""
    m, h, d = q.shape
    hkv = k.shape[1]
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2).repeat_interleave(h // hkv, 0)
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2).repeat_interleave(h // hkv, 0)
    mask = None if vis is None else torch.from_numpy(vis)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    return o.permute(1, 0, 2).numpy()


@pytest.mark.parametrize("m,n,h,hkv", [(1, 256, 24, 4), (1, 1000, 48, 8), (5, 300, 4, 2), (3, 64, 4, 4)])
def test_attention_vs_torch_sdpa(m, n, h, hkv):
    rng = np.random.default_rng(m * 1000 + n)
    q = rng.standard_normal((m, h, 256)).astype(np.float16)
    k = rng.standard_normal((n, hkv, 256)).astype(np.float16)
    v = rng.standard_normal((n, hkv, 256)).astype(np.float16)
    got = orc.attention_fp32(q, k, v)
    assert np.max(np.abs(got - _sdpa64(q, k, v))) < 1e-5


def test_attention_special_cases():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 24, 256)).astype(np.float16)
    v = rng.standard_normal((7, 4, 256)).astype(np.float16)
    # L = 1: the output is v_0.
    out = orc.attention_fp32(q, rng.standard_normal((1, 4, 256)).astype(np.float16), v[:1])
    assert np.array_equal(out[0], np.repeat(v[0].astype(np.float32), 6, 0))
    # Identical keys: the output is the mean of V.
    k = np.repeat(rng.standard_normal((1, 4, 256)).astype(np.float16), 7, 0)
    out = orc.attention_fp32(q, k, v)
    assert np.allclose(out[0], np.repeat(v.astype(np.float32).mean(0), 6, 0), atol=1e-6)
    # One dominant key (score +80 vs 0): the output is that key's V row.
    k = np.zeros((7, 4, 256), np.float16)
    qq = np.zeros((1, 24, 256), np.float16)
    qq[..., 0] = 32
    k[3, :, 0] = 40  # score = 32*40/16 = 80
    out = orc.attention_fp32(qq, k, v)
    assert np.allclose(out[0], np.repeat(v[3].astype(np.float32), 6, 0), atol=1e-6)


def test_gqa_head_map():
    # flash_attn_256_tuned.hip:222: kv = h*Hkv/H; equals h // (H/Hkv).
    for h_total, hkv in [(24, 4), (48, 8), (4, 2), (8, 2), (4, 4)]:
        for h in range(h_total):
            assert orc.kv_head_of(h, h_total, hkv) == h // (h_total // hkv)


def test_split_merge_matches_single_pass():
    rng = np.random.default_rng(2)
    q = rng.standard_normal(256)
    k = rng.standard_normal((1000, 256))
    v = rng.standard_normal((1000, 256))
    full = orc.merge_partials(*[np.array(x) for x in zip(orc.partial_softmax(q, k, v))])
    for cuts in ([0, 1000], [0, 64, 1000], [0, 17, 500, 999, 1000]):
        parts = [orc.partial_softmax(q, k[a:b], v[a:b]) for a, b in zip(cuts[:-1], cuts[1:])]
        ms, ls, accs = zip(*parts)
        assert np.allclose(orc.merge_partials(ms, ls, np.stack(accs)), full, atol=1e-12)
    s = k @ q / 16
    p = np.exp(s - s.max())
    assert np.allclose(full, p @ v / p.sum(), atol=1e-12)


def test_chunk_causal_rules():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((6, 4, 256)).astype(np.float16)
    k = rng.standard_normal((10, 2, 256)).astype(np.float16)
    v = rng.standard_normal((10, 2, 256)).astype(np.float16)
    # prefix 0: the reference's causal rule == torch's is_causal.
    got = orc.chunk_attention(q, k[:6], v[:6], 0)
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)
    kt = torch.from_numpy(k[:6].astype(np.float64)).permute(1, 0, 2).repeat_interleave(2, 0)
    vt = torch.from_numpy(v[:6].astype(np.float64)).permute(1, 0, 2).repeat_interleave(2, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True)
    assert np.max(np.abs(got - ref.permute(1, 0, 2).numpy())) < 1e-5
    # prefix 4: chunk row i sees 5+i keys; the last row is plain decode.
    got = orc.chunk_attention(q, k, v, 4)
    for i in range(6):
        row = orc.attention_fp32(q[i:i + 1], k[:5 + i], v[:5 + i])[0]
        assert np.allclose(got[i], row, atol=1e-6)


# ------------------------------------------------------------------ tree (a10)
def test_tree_mask_known_answers():
    g = golden()
    m3 = orc.tree_mask_reference(g["tree3_parents"], g["tree3_kv_len"]).astype(int)
    assert m3.tolist() == g["tree3_rows"]
    m7 = orc.tree_mask_reference(g["tree7_parents"], g["tree7_kv_len"]).astype(int)
    assert m7.shape == (7, 9)
    assert m7[0].tolist() == g["tree7_row0"] and m7[3].tolist() == g["tree7_row3"]
    counts = [len(orc.tree_ancestors(g["tree7_parents"], i)) + 1 for i in range(7)]
    assert counts == g["tree7_ancestor_counts"]


def test_tree_depths_pinned():
    """oracle.tree_depths, the RoPE offset of tree rows (position len + depth):
    the depths the reference's own tests assert, config 5's tree, and closed
    forms (a chain is arange; a complete binary tree in BFS order puts node i
    at floor(log2(i + 1))).  Depth as the number of ancestors is checked too,
    so an off-by-one (root at 1) or a parent-index mix-up fails."""
    for case in golden()["tree_depth_cases"]:
        d = orc.tree_depths(case["parents"]).tolist()
        if "depths" in case:
            assert d == case["depths"]
        if "max_depth" in case:
            assert max(d) == case["max_depth"]
        if "nodes_per_depth" in case:
            assert [d.count(k) for k in range(max(d) + 1)] == case["nodes_per_depth"]
    assert orc.tree_depths([-1, 0, 0, 0, 1, 1, 2, 4, 4]).tolist() == [0, 1, 1, 1, 2, 2, 2, 3, 3]
    assert orc.tree_depths([-1] + list(range(11))).tolist() == list(range(12))
    binary = [-1] + [(i - 1) // 2 for i in range(1, 63)]
    assert orc.tree_depths(binary).tolist() == [int(np.floor(np.log2(i + 1))) for i in range(63)]
    rng = np.random.default_rng(3)
    for _ in range(50):
        n = int(rng.integers(1, 40))
        parents = [-1] + [int(rng.integers(0, i)) for i in range(1, n)]
        assert orc.tree_depths(parents).tolist() == [len(orc.tree_ancestors(parents, i)) for i in range(n)]
    with pytest.raises(AssertionError):
        orc.tree_depths([0, 0])        # no root
    with pytest.raises(AssertionError):
        orc.tree_depths([-1, 2, 0])    # a parent after its child


def test_tree_mask_invariants_and_cache_order():
    parents = [-1, 0, 0, 0, 1, 1, 2, 4, 4]
    m = orc.tree_mask_reference(parents, 5)
    t = len(parents)
    for i in range(t):
        anc = set(orc.tree_ancestors(parents, i)) | {i}
        assert {j for j in range(t) if m[i, j]} == anc           # self + ancestors only
        assert all(j <= i for j in anc)                            # BFS lower triangular
        assert m[i, t:].all()                                      # all KV visible
    c = orc.tree_visibility_cache_order(parents, 5)
    assert np.array_equal(c[:, :5], m[:, t:]) and np.array_equal(c[:, 5:], m[:, :t])
    bits = orc.tree_row_bits(parents)
    for i in range(t):
        assert [(int(bits[i]) >> j) & 1 for j in range(t)] == m[i, :t].astype(int).tolist()


def test_chain_tree_equals_causal():
    # tests/test_tree_vs_causal_attention.py:177-218: a chain tree is causal.
    rng = np.random.default_rng(42)
    parents = [-1, 0, 1, 2, 3]
    q = rng.standard_normal((5, 4, 256)).astype(np.float16)
    kc = rng.standard_normal((3, 2, 256)).astype(np.float16)
    vc = rng.standard_normal((3, 2, 256)).astype(np.float16)
    kt = rng.standard_normal((5, 2, 256)).astype(np.float16)
    vt = rng.standard_normal((5, 2, 256)).astype(np.float16)
    tree = orc.tree_attention(q, kc, vc, kt, vt, parents)
    causal = orc.chunk_attention(q, np.concatenate([kc, kt]), np.concatenate([vc, vt]), 3)
    assert np.max(np.abs(tree - causal)) < 1e-6
    # A branching tree differs from causal (node 2 must not see node 1).
    tree_b = orc.tree_attention(q, kc, vc, kt, vt, [-1, 0, 0, 1, 2])
    assert np.max(np.abs(tree_b[2] - causal[2])) > 1e-4


def test_rollback_semantics():
    rows = np.arange(20)
    out, n = orc.rollback_rows(rows, 10, [0, 2, 3])
    assert n == 13
    assert out[:10].tolist() == list(range(10))                 # prefix untouched
    assert out[10:13].tolist() == [10, 12, 13]                   # accepted rows compacted
    assert out[13:].tolist() == list(range(13, 20))              # beyond the length: as before
    with pytest.raises(AssertionError):
        orc.rollback_rows(rows, 10, [2, 1])


def test_paged_model_gather_is_layout_independent():
    rng = np.random.default_rng(8)
    a = orc.PagedCacheModel(1, 12, num_kv_heads=2, head_dim=16)
    b = orc.PagedCacheModel(1, 12, num_kv_heads=2, head_dim=16)
    a.set_table(0, [5, 0, 9])
    b.set_table(0, [1, 2, 3])
    rows = rng.standard_normal((40, 2, 2, 16)).astype(np.float16)
    for s in range(40):
        a.write(0, 0, s, rows[s, 0], rows[s, 1])
        b.write(0, 0, s, rows[s, 0], rows[s, 1])
    ka, va = a.gather(0, 0, 40)
    kb, vb = b.gather(0, 0, 40)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    assert np.array_equal(ka, rows[:, 0])
    assert np.array_equal(a.k[0, 9, 7], rows[39, 0])             # slot 39 -> block 9 row 7


# ------------------------------------------------------------ planted mistakes
def test_planted_mistakes_are_caught():
    """Mutated oracles must fail the pins above (mistakes planted on the CPU)."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 256)).astype(np.float16)
    w = (1 + 0.02 * rng.standard_normal(256)).astype(np.float16)
    cos, sin = orc.rope_tables(1000)
    pos = rng.integers(1, 1000, 8)
    ref = _norm_rope_f64(x, w, cos[pos].astype(np.float64), sin[pos].astype(np.float64))

    def rotate_half(x, w, c, s):  # HF convention instead of interleaved pairs
        n = _norm_rope_f64(x, w, np.ones_like(c, dtype=np.float64), np.zeros_like(s, dtype=np.float64))
        a, b = n[:, :32].copy(), n[:, 32:64].copy()
        n[:, :32] = a * c - b * s
        n[:, 32:64] = a * s + b * c
        return n

    def sign_flip(x, w, c, s):
        return orc.qknorm_rope_exact(x, w, c, (-s.astype(np.float32)).astype(np.float16))

    for bad in (rotate_half, sign_flip):
        got = np.asarray(bad(x, w, cos[pos], sin[pos]), dtype=np.float64)
        assert np.max(np.abs(got - ref)) > 1e-2, bad.__name__

    q = rng.standard_normal((1, 24, 256)).astype(np.float16)
    k = rng.standard_normal((50, 4, 256)).astype(np.float16)
    v = rng.standard_normal((50, 4, 256)).astype(np.float16)
    good = _sdpa64(q, k, v)
    # Wrong GQA map (h % Hkv) and missing 1/sqrt(d) both fail the torch pin.
    k_mod = k[:, [0, 1, 2, 3]]
    wrong_map = np.stack([orc.attention_fp32(q[:, h:h + 1], k_mod[:, h % 4:h % 4 + 1],
                                             v[:, h % 4:h % 4 + 1])[:, 0] for h in range(24)], 1)
    assert np.max(np.abs(wrong_map - good)) > 1e-2
    no_scale = orc.attention_fp32((q.astype(np.float32) * 16).astype(np.float16), k, v)
    assert np.max(np.abs(no_scale - good)) > 1e-2
    # Tree-first columns used as cache-first columns fail the known answers.
    g = golden()
    swapped = orc.tree_visibility_cache_order(g["tree3_parents"], g["tree3_kv_len"]).astype(int)
    assert swapped.tolist() != g["tree3_rows"]


def test_sigmoid_gate_pins():
    """sigmoid_mul.hip:10-22 restated: closed-form gates, the sigmoid's
    symmetry, and a float64 computation within one fp16 rounding."""
    rng = np.random.default_rng(9)
    out = (rng.standard_normal(4096) * 3).astype(np.float16)
    out = out[np.abs(out.astype(np.float32)) > 1e-3]  # normal range: halving is exact
    z = np.zeros_like(out)
    assert np.array_equal(orc.sigmoid_gate(out, z).view(np.uint16), (out / np.float16(2)).view(np.uint16))
    assert np.array_equal(orc.sigmoid_gate(out, z + np.float16(20)).view(np.uint16), out.view(np.uint16))
    assert np.all(orc.sigmoid_gate(out, z - np.float16(20)).astype(np.float32) == 0)
    g = (rng.standard_normal(out.shape) * 2).astype(np.float16)
    both = orc.sigmoid_gate(out, g).astype(np.float32) + orc.sigmoid_gate(out, -g).astype(np.float32)
    ulp = np.abs(out.astype(np.float32)) * 2.0 ** -10
    assert np.all(np.abs(both - out.astype(np.float32)) <= 2 * ulp + 1e-7)
    ref = (out.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))).astype(np.float16)
    diff = np.abs(orc.sigmoid_gate(out, g).astype(np.float64) - ref.astype(np.float64))
    assert np.all(diff <= np.abs(ref.astype(np.float64)) * 2.0 ** -10 + 1e-7)


# ---------------------------------------------------------------- projection
def _project_fraction(x, w):
    """Exact rational sum per output, then one fp16 rounding (brute force)."""
    from fractions import Fraction

    T, K = x.shape
    N = w.shape[0]
    out = np.empty((T, N), np.float16)
    for t in range(T):
        xs = [Fraction(float(v)) for v in x[t]]
        for n in range(N):
            acc = sum((Fraction(float(w[n, k])) * xs[k] for k in range(K)), Fraction(0))
            out[t, n] = np.float16(float(acc))
    return out


def test_project_fp16_pins():
    """gemv_fp16_v2.hip:22-85 restated: exact rational brute force on small
    cases (a transposed operand or a dropped term fails it), unit rows pick
    single elements, and fp32-exact integer sums survive any order."""
    rng = np.random.default_rng(5)
    for T, K, N in ((1, 64, 8), (3, 32, 5), (2, 96, 7)):
        x = rng.standard_normal((T, K)).astype(np.float16)
        w = (rng.standard_normal((N, K)) * 0.2).astype(np.float16)
        assert np.array_equal(orc.project_fp16(x, w).view(np.uint16), _project_fraction(x, w).view(np.uint16))
        assert not np.array_equal(orc.project_fp16(x, w[::-1]), _project_fraction(x, w))
    x = rng.standard_normal((4, 512)).astype(np.float16)
    pick = rng.integers(0, 512, 40)
    w = np.zeros((40, 512), np.float16)
    w[np.arange(40), pick] = 1
    assert np.array_equal(orc.project_fp16(x, w).view(np.uint16), x[:, pick].view(np.uint16))
    # Integer products of magnitude <= 6 * 2^-7 summed over 5120 terms stay
    # exact in fp32: the sum is order independent and equals the fp32 sum.
    xi = rng.integers(-3, 4, (2, 5120)).astype(np.float16)
    wi = (rng.integers(-2, 3, (16, 5120)) * 2.0 ** -7).astype(np.float16)
    f32 = np.zeros((2, 16), np.float32)
    for k in range(0, 5120, 512):
        f32 += xi[:, k:k + 512].astype(np.float32) @ wi[:, k:k + 512].astype(np.float32).T
    assert np.array_equal(orc.project_fp16(xi, wi).view(np.uint16), f32.astype(np.float16).view(np.uint16))


def test_out_project_pins():
    """The O-projection's residual epilogue (gemv_fp16_v2.hip:81-84): exact
    rational brute force with the residual inside the one rounding (adding
    it after a first rounding fails), no residual is project_fp16, a zero
    weight returns the residual bit for bit, and unit rows add one element."""
    from fractions import Fraction

    rng = np.random.default_rng(15)
    T, K, N = 3, 64, 9
    x = rng.standard_normal((T, K)).astype(np.float16)
    w = (rng.standard_normal((N, K)) * 0.2).astype(np.float16)
    r = rng.standard_normal((T, N)).astype(np.float16)
    want = np.empty((T, N), np.float16)
    for t in range(T):
        for n in range(N):
            acc = sum((Fraction(float(w[n, k])) * Fraction(float(x[t, k])) for k in range(K)),
                      Fraction(float(r[t, n])))
            want[t, n] = np.float16(float(acc))
    got = orc.out_project(x, w, r)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    big = rng.standard_normal((64, 512)).astype(np.float16)
    wb = (rng.standard_normal((48, 512)) * 0.05).astype(np.float16)
    rb = (rng.standard_normal((64, 48)) * 30).astype(np.float16)
    twice_b = (orc.project_fp16(big, wb).astype(np.float32) + rb.astype(np.float32)).astype(np.float16)
    assert not np.array_equal(orc.out_project(big, wb, rb), twice_b)
    assert np.array_equal(orc.out_project(x, w).view(np.uint16), orc.project_fp16(x, w).view(np.uint16))
    assert np.array_equal(orc.out_project(x, np.zeros_like(w), r).view(np.uint16), r.view(np.uint16))
    pick = rng.integers(0, K, N)
    wu = np.zeros((N, K), np.float16)
    wu[np.arange(N), pick] = 1
    sums = (x[:, pick].astype(np.float64) + r.astype(np.float64)).astype(np.float16)
    assert np.array_equal(orc.out_project(x, wu, r).view(np.uint16), sums.view(np.uint16))


def test_project_append_layout():
    """The producer composite reads the stacked weights the reference's way
    (engine.py:1366-1378: Q rows then Q_gate rows, K rows then V rows) and
    hands Q and K to the pinned norm + RoPE.  Unit-row weights make every
    projected value a known element of x, so a swapped half or head order
    shows up as a wrong element."""
    rng = np.random.default_rng(6)
    H, HKV, D, K, T = 2, 1, 256, 512, 3
    x = rng.standard_normal((T, K)).astype(np.float16)
    wq = np.zeros((2 * H * D, K), np.float16)
    wkv = np.zeros((2 * HKV * D, K), np.float16)
    sq = rng.integers(0, K, 2 * H * D)
    skv = rng.integers(0, K, 2 * HKV * D)
    wq[np.arange(2 * H * D), sq] = 1
    wkv[np.arange(2 * HKV * D), skv] = 1
    qw = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
    kw = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
    cos, sin = orc.rope_tables(64)
    pos = np.array([5, 17, 40])
    q, gate, k_raw, k, v = orc.project_append(x, wq, wkv, qw, kw, cos[pos], sin[pos], H, HKV)
    q_raw = x[:, sq[:H * D]].reshape(T, H, D)
    assert np.array_equal(gate.view(np.uint16), x[:, sq[H * D:]].reshape(T, H, D).view(np.uint16))
    assert np.array_equal(k_raw.view(np.uint16), x[:, skv[:HKV * D]].reshape(T, HKV, D).view(np.uint16))
    assert np.array_equal(v.view(np.uint16), x[:, skv[HKV * D:]].reshape(T, HKV, D).view(np.uint16))
    for h in range(H):
        exp = orc.qknorm_rope_exact(q_raw[:, h], qw, cos[pos], sin[pos])
        assert np.array_equal(q[:, h].view(np.uint16), exp.view(np.uint16))
    exp = orc.qknorm_rope_exact(k_raw[:, 0], kw, cos[pos], sin[pos])
    assert np.array_equal(k[:, 0].view(np.uint16), exp.view(np.uint16))
