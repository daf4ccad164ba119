"""Pins the oracle's RWKV-7 step (CPU only).

- The reference's own element-wise accuracy tests, with their inputs and bounds
  (src/domain/tensor.rs:2372-2500), and its rank-1 identity test (:2502-2537).
- Closed forms: GroupNorm of a constant group, the l2-norm guard, the WKV recurrence on
  a single head against the explicit matrix form in float64.
- The whole step against an independent float64 model (tests/rwkv_f64.py) over several
  tokens, F32 and int8 weight-only, with a plausible mistake planted in the oracle
  shown to fail the same comparison.
- Lockstep == single stream bit for bit, thread-count independence, reset == fresh.
- The weight container and the BlinkDL import.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import rwkv
from tests.rwkv_f64 import F64Rwkv

SMALL = rwkv.RwkvDims(vocab=300, d_model=128, n_layer=2, head_size=64, d_ffn=256, lora_w=16, lora_a=16,
                      lora_v=8, lora_g=32)


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def bits(a):
    return f32(a).view(np.uint32)


def call(name, *arrays_and_ints):
    args = [O._p(a) if isinstance(a, np.ndarray) else a for a in arrays_and_ints]
    getattr(O.lib(), name)(*args)


# ---- element-wise: the reference's accuracy tests (tensor.rs:2372-2500) ----

def exact_sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def test_sigmoid_inplace_accuracy():
    x = f32([i * 0.25 for i in range(-40, 41)])
    y = x.copy()
    call("orc_sigmoid_inplace", y, y.size)
    assert np.max(np.abs(y - exact_sigmoid(x))) < 2e-7


def test_tanh_inplace_accuracy():
    x = f32([i * 0.25 for i in range(-40, 41)])
    y = x.copy()
    call("orc_tanh_inplace", y, y.size)
    assert np.max(np.abs(y - np.tanh(x.astype(np.float64)))) < 5e-7


def _ref_vectors(n=768):
    i = np.arange(n, dtype=np.float32)
    base = f32(np.sin(i * np.float32(0.013)) * 4.0)
    offset = f32(np.cos(i * np.float32(0.007)) * 3.0)
    return base, offset


def test_sigmoid_add_into_accuracy():
    base, offset = _ref_vectors()
    out = np.empty_like(base)
    call("orc_sigmoid_add_into", out, base, offset, base.size)
    assert np.max(np.abs(out - exact_sigmoid(base.astype(np.float64) + offset))) < 2e-7


def test_decay_sigmoid_into_accuracy():
    base, offset = _ref_vectors()
    out = np.empty_like(base)
    call("orc_decay_sigmoid_into", out, base, offset, base.size)
    expected = np.exp(-0.606531 * exact_sigmoid(base.astype(np.float64) + offset))
    assert np.max(np.abs(out - expected)) < 5e-7


def test_sigmoid_mix_inplace_accuracy():
    base, offset = _ref_vectors()
    i = np.arange(768, dtype=np.float32)
    v_first = f32(np.sin(i * np.float32(0.019)) * 2.0)
    v = f32(np.cos(i * np.float32(0.011)) * 1.5)
    out = v.copy()
    call("orc_sigmoid_mix_inplace", out, v_first, base, offset, 768)
    mix = exact_sigmoid(base.astype(np.float64) + offset)
    assert np.max(np.abs(out - (v + (v_first - v) * mix))) < 5e-7


@pytest.mark.parametrize("fn,exact,bound", [("orc_sigmoid_inplace", exact_sigmoid, 2e-7),
                                            ("orc_tanh_inplace", np.tanh, 5e-7)])
def test_boundary_values(fn, exact, bound):
    x = f32([-100.0, -50.0, -10.0, -1.0, 0.0, 1.0, 10.0, 50.0, 100.0])
    y = x.copy()
    call(fn, y, y.size)  # 9 elements: 8-lane body plus a portable tail element
    assert np.max(np.abs(y - exact(x.astype(np.float64)))) < bound


def test_rank1_factorisation():
    """tensor.rs:2502-2537: S·outer(u, v) against outer(S·u, v), same inputs and bound."""
    n = 64
    i = np.arange(n * n, dtype=np.float32)
    state = f32(np.sin(i * np.float32(0.007)) * 2.0)
    u = f32(np.cos(np.arange(n, dtype=np.float32) * np.float32(0.013)) * 1.5)
    v = f32(np.sin(np.arange(n, dtype=np.float32) * np.float32(0.019)) * 1.0)
    temp = np.empty(n, np.float32)
    call("orc_mat_vec_small", temp, state, u, n)
    factored = np.outer(temp, v).astype(np.float32)
    original = state.reshape(n, n).astype(np.float64) @ np.outer(u, v).astype(np.float64)
    assert np.max(np.abs(factored - original)) < 1e-4


# ---- closed forms ----

def test_group_norm_constant_group_gives_bias():
    x = np.concatenate([np.full(64, 3.5, np.float32), np.arange(64, dtype=np.float32)])
    w, b = f32(np.linspace(0.5, 2.0, 128)), f32(np.linspace(-1.0, 1.0, 128))
    out = np.empty(128, np.float32)
    call("orc_group_norm_into", out, x, 2, w, b, 128, ctypes.c_float(64e-5))
    assert np.array_equal(out[:64], b[:64])           # x - mean == 0 exactly
    g = np.arange(64, dtype=np.float64)
    ref = (g - g.mean()) / np.sqrt(g.var() + 64e-5) * w[64:] + b[64:]
    assert np.max(np.abs(out[64:] - ref)) < 2e-6


def test_l2_norm_guard_and_unit_norm():
    x = np.zeros(128, np.float32)
    x[64:] = np.arange(1, 65, dtype=np.float32)
    call("orc_l2_normalize_per_head", x, 2, 64)
    assert np.all(x[:64] == 0.0)                       # norm 0 <= 1e-12 -> inv 0
    assert abs(float(np.linalg.norm(x[64:].astype(np.float64))) - 1.0) < 1e-6


def test_wkv_head_against_matrix_form():
    rng = np.random.default_rng(5)
    n = 64
    S0 = f32(rng.normal(0, 0.5, (n, n)))
    r, kk_raw, v = (f32(rng.normal(0, 1, n)) for _ in range(3))
    kk = f32(kk_raw / np.linalg.norm(kk_raw))
    w = f32(rng.uniform(0.9, 0.999, n))
    a = f32(rng.uniform(0, 1, n))
    kmod = f32(rng.normal(0, 1, n))
    S = S0.copy()
    out = np.empty(n, np.float32)
    tmp = np.empty(3 * n, np.float32)
    for _ in range(3):
        call("orc_wkv_head", S, n, r, w, kk, a, v, kmod, out, tmp)
    E = S0.astype(np.float64)
    for _ in range(3):
        E = E @ np.diag(w.astype(np.float64)) + E @ np.outer(-kk, kk * a) + np.outer(v, kmod)
    assert np.max(np.abs(S - E)) < 1e-5
    assert np.max(np.abs(out - E @ r)) < 1e-4
    # a wrong index (state transposed in the update) must not pass the same bound
    bad = S0.astype(np.float64).T @ np.diag(w) + S0.T @ np.outer(-kk, kk * a) + np.outer(v, kmod)
    one = S0.copy()
    call("orc_wkv_head", one, n, r, w, kk, a, v, kmod, out, tmp)
    assert np.max(np.abs(one - bad)) > 1e-3


# ---- the whole step against float64 ----

@pytest.fixture(scope="module")
def small_model(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("rwkv") / "small.rbin")
    rwkv.write_synthetic(p, SMALL, seed=1)
    return p


def dequantized(path, dims, group):
    _, t = rwkv.read_rwkv(path)
    mats = {}
    names = ["head"] + [f"blocks.{i}.{m}" for i in range(dims.n_layer)
                        for m in ("receptance", "key", "value", "output", "ffn_key", "ffn_value")]
    for name in names:
        w = f32(t[name])
        g = w.shape[1] if group == 0 else group
        q, sc, g = O.quantize(w, g)
        mats[name] = (q.astype(np.float32).reshape(w.shape[0], -1, g) * sc.reshape(w.shape[0], -1, 1)).reshape(w.shape)
    return mats


def run_compare(path, dims, profile, tokens, slots=(0, 1)):
    orc = O.RwkvOracle(path, profile, cap=len(slots))
    _, t = rwkv.read_rwkv(path)
    group = {0: None, 1: 64, 2: 0}[profile & 3]
    ref = F64Rwkv(dims, t, dequantized(path, dims, group) if group is not None else None)
    worst = 0.0
    for step in tokens:
        lo = orc.forward(list(slots), list(step))
        for b, s in enumerate(slots):
            e = ref.step(s, step[b])
            worst = max(worst, float(np.max(np.abs(lo[b] - e))))
    orc.close()
    return worst


TOKENS = [[5, 17], [250, 3], [17, 17], [0, 299], [42, 7], [8, 9]]
STEP_TOL = 1e-6   # max |logit(oracle) - logit(float64)| over TOKENS


@pytest.mark.parametrize("profile", [0, 1, 2])
def test_step_matches_float64(small_model, profile):
    worst = run_compare(small_model, SMALL, profile, TOKENS)
    assert worst < STEP_TOL, worst


def test_planted_mistake_fails_float64(small_model, tmp_path):
    """The float64 comparison has teeth: an oracle built with the bonus term taken from
    the modified key instead of the key (a one-word change) fails it."""
    src = os.path.dirname(os.path.abspath(O.__file__))
    text = open(os.path.join(src, "rwkv7_oracle.c")).read()
    planted = text.replace("const float* ksrc = m->g1k ? s->kmod : s->k;", "const float* ksrc = s->kmod;")
    assert planted != text
    (tmp_path / "rwkv7_oracle.c").write_text(planted)
    lib = str(tmp_path / "liboracle_planted.so")
    subprocess.run(["gcc", "-O2", "-std=gnu11", "-fPIC", "-ffp-contract=off", "-shared", "-pthread", f"-I{src}",
                    os.path.join(src, "mamba_oracle.c"), str(tmp_path / "rwkv7_oracle.c"), os.path.join(src, "pool.c"),
                    "-o", lib, "-lm"], check=True)
    root = os.path.dirname(src)
    code = ("from tests.test_oracle_rwkv import run_compare, SMALL, TOKENS; "
            f"print(run_compare({small_model!r}, SMALL, 0, TOKENS))")
    res = subprocess.run(["python3", "-c", code], cwd=root, env={**os.environ, "ORACLE_LIB": lib},
                         capture_output=True, text=True, check=True)
    worst = float(res.stdout.strip().splitlines()[-1])
    assert worst > 4 * STEP_TOL, worst


# ---- invariants ----

@pytest.mark.parametrize("profile", [0, 2])
def test_lockstep_bit_identical_to_single_stream(small_model, profile):
    m = O.RwkvOracle(small_model, profile, cap=5)
    n, steps = 5, 4
    toks = [[(s * 37 + t * 101 + 3) % m.vocab for t in range(steps)] for s in range(n)]
    ref = []
    for s in range(n):
        m.reset()
        for t in range(steps):
            lo = m.forward([0], [toks[s][t]])
        ref.append((lo[0].copy(), [m.state(0, l) for l in range(m.n_layer)]))
    m.reset()
    order = [3, 0, 4, 1, 2]                    # slot s runs at batch position order.index(s)
    for t in range(steps):
        lo = m.forward(order, [toks[s][t] for s in order])
    for b, s in enumerate(order):
        assert np.array_equal(bits(lo[b]), bits(ref[s][0])), (profile, s)
        for l in range(m.n_layer):
            for got, want in zip(m.state(s, l), ref[s][1][l]):
                assert np.array_equal(bits(got), bits(want))
    m.close()


def test_threads_do_not_change_bits(small_model):
    outs = []
    for th in (1, 3, 8):
        O.set_threads(th)
        m = O.RwkvOracle(small_model, 2, cap=6)
        for t in range(3):
            lo = m.forward(list(range(6)), [(b * 7 + t) % m.vocab for b in range(6)])
        outs.append(lo.copy())
        m.close()
    O.set_threads(0)
    assert all(np.array_equal(bits(o), bits(outs[0])) for o in outs)


def test_reset_equals_fresh_and_periodic(small_model):
    m = O.RwkvOracle(small_model, 0, cap=2)
    for t in range(3):
        m.forward([0, 1], [t, t + 1])
    m.reset([1])
    fresh = O.RwkvOracle(small_model, 0, cap=1)
    a = m.forward([1], [11])
    b = fresh.forward([0], [11])
    assert np.array_equal(bits(a), bits(b))
    # period 3: the 4th forward of a slot runs on zero state
    m.reset()
    m.set_reset_every(3)
    for t in range(3):
        m.forward([0], [t + 20])
    after = m.forward([0], [11])
    assert np.array_equal(bits(after), bits(b))
    m.close()
    fresh.close()


def test_invalid_arguments(small_model):
    m = O.RwkvOracle(small_model, 0, cap=2)
    for slots, toks in (([0, 0], [1, 2]), ([2], [1]), ([0], [m.vocab]), ([0, 1, 1], [1, 2, 3])):
        with pytest.raises(ValueError):
            m.forward(slots, toks)
    m.close()


# ---- the weight container ----

def test_container_round_trip_and_header(small_model, tmp_path):
    dims, t = rwkv.read_rwkv(small_model)
    assert dims == SMALL
    assert os.path.getsize(small_model) == rwkv.file_bytes(SMALL)
    with open(small_model, "rb") as f:
        head = f.read(64)
    assert rwkv.parse_header(head) == SMALL
    from redukt_amd import rbin
    assert rbin.parse_rbin_header(head) is None   # the Mamba host reader ignores it
    bad = bytearray(head)
    bad[8] = 1                                   # model word != RWKV-7
    assert rwkv.parse_header(bytes(bad)) is None
    short = tmp_path / "short.rbin"
    short.write_bytes(open(small_model, "rb").read()[:-4])
    with pytest.raises(RuntimeError):
        O.RwkvOracle(str(short), 0)


def test_blinkdl_import_matches_direct_write(tmp_path):
    """A BlinkDL-named tensor set (as rwkv7/model.rs:997-1059 reads it) converts to the
    same tensors: ln0 applied to the embedding, LoRAs transposed, r_k flattened."""
    dims = SMALL
    rng = np.random.default_rng(3)
    t = rwkv.synthetic(dims, seed=4)
    raw_emb = f32(rng.normal(0, 1, (dims.vocab, dims.d_model)))
    ln0_w, ln0_b = f32(rng.uniform(0.5, 1.5, dims.d_model)), f32(rng.normal(0, 0.1, dims.d_model))
    blink = {"emb.weight": raw_emb, "blocks.0.ln0.weight": ln0_w, "blocks.0.ln0.bias": ln0_b,
             "ln_out.weight": t["ln_out_w"], "ln_out.bias": t["ln_out_b"], "head.weight": t["head"]}
    H, N = dims.n_head, dims.head_size
    for i in range(dims.n_layer):
        p, att, ffn = f"blocks.{i}.", f"blocks.{i}.att.", f"blocks.{i}.ffn."
        blink[p + "ln1.weight"], blink[p + "ln1.bias"] = t[p + "ln1_w"], t[p + "ln1_b"]
        blink[p + "ln2.weight"], blink[p + "ln2.bias"] = t[p + "ln2_w"], t[p + "ln2_b"]
        for name in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "a0", "v0", "k_k", "k_a"):
            blink[att + name] = t[p + name].reshape(1, 1, -1)
        for name in ("w1", "w2", "a1", "a2", "v1", "v2", "g1", "g2"):
            blink[att + name] = np.ascontiguousarray(t[p + name].T)
        blink[att + "r_k"] = t[p + "r_k"].reshape(H, N)
        for name in ("receptance", "key", "value", "output"):
            blink[att + name + ".weight"] = t[p + name]
        blink[att + "ln_x.weight"], blink[att + "ln_x.bias"] = t[p + "ln_x_w"], t[p + "ln_x_b"]
        blink[ffn + "x_k"] = t[p + "ffn_x_k"].reshape(1, 1, -1)
        blink[ffn + "key.weight"], blink[ffn + "value.weight"] = t[p + "ffn_key"], t[p + "ffn_value"]
    dims2, conv = rwkv.from_blinkdl(blink, dims.n_layer, head_size=N)
    assert dims2 == dims
    for name, _ in rwkv.tensor_order(dims):
        if name == "emb":
            continue
        assert np.array_equal(conv[name], t[name]), name
    # ln0 in the reference's f32 order, checked against float64
    e64 = raw_emb.astype(np.float64)
    mu = e64.mean(axis=1, keepdims=True)
    ref = (e64 - mu) / np.sqrt(((e64 - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5) * ln0_w + ln0_b
    assert np.max(np.abs(conv["emb"] - ref)) < 2e-5
