"""Plans on the CPU (no GPU needed): workspace placement never overlaps live values, layout ops feeding
dots are strided views, and every generated loop kernel compiles for gfx950 with hipcc."""

import numpy as np
import pytest

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd import workloads as W
from lumen_amd.compiler.plan import Plan
from lumen_amd.graph.trace import trace


def _plan(fn, *metas, build=False):
    g = L.make_graph(fn)(*[L.empty(list(s), d, "meta") for s, d in metas])
    return Plan(g, build_kernels=build)


def test_placement_never_overlaps_live_values():
    model, opt = W.build(W.TINY)
    ids = L.empty([W.TINY.batch, W.TINY.seq], "int64", "meta")
    p = Plan(trace(W.train_step, (model, opt, ids, ids)).graph, build_kernels=False)
    g = p.graph
    first, last = {}, {}
    for si, st in enumerate(p.steps):
        for v in st.outputs:
            first.setdefault(v, si)
        for u in st.inputs:
            last[u] = si
    for v in g.outputs:
        last[v] = len(p.steps)
    spans = []
    for v, si in first.items():
        loc = p.loc[v]
        if loc.base[0] != "ws" or p.steps[si].kind == "view":
            continue
        start = loc.offset * g.types[v].nbytes() // max(1, g.types[v].numel())
        spans.append((si, last.get(v, si), start, start + g.types[v].nbytes(), v))
    for a in spans:
        for b in spans:
            if a[4] < b[4] and a[0] <= b[1] and b[0] <= a[1]:
                assert a[3] <= b[2] or b[3] <= a[2], (a, b)
    assert p.workspace_bytes % 256 == 0


def test_transposed_weight_feeds_the_dot_as_a_view():
    """A transposed graph input feeding a dot folds into the dot's dimension numbers (simplify), and the
    GEMM reads the weight in its stored [n, k] layout: no copy and no view step."""
    p = _plan(lambda x, w: F.matmul(x, w.t(), "float32", "bfloat16"), ((64, 32), "bfloat16"), ((48, 32), "bfloat16"))
    assert [s.kind for s in p.steps] == ["dot"]
    desc, ops = p._gemm_desc(p.steps[0].nodes[0])
    assert (desc.m, desc.n, desc.k, desc.b_k, desc.b_n) == (64, 48, 32, 1, 32)


def test_concatenated_dot_results_are_written_in_place():
    """Two dot results only read by a concatenation are placed inside it as strided views: the
    concatenation launches nothing, and the consuming dot reads the one buffer."""
    def fn(x, w1, w2, w3):
        a = F.matmul(x, w1, "float32", "bfloat16")
        b = F.matmul(x, w2, "float32", "bfloat16")
        return F.matmul(F.cat([a, b], 1), w3, "float32", "bfloat16")

    p = _plan(fn, ((2048, 256), "bfloat16"), ((256, 512), "bfloat16"), ((256, 512), "bfloat16"),
              ((1024, 128), "bfloat16"))
    kinds = [s.kind for s in p.steps]
    assert kinds == ["dot", "dot", "alias", "dot"], kinds
    a, b = p.steps[0].outputs[0], p.steps[1].outputs[0]
    c = p.steps[2].outputs[0]
    la, lb, lc = p.loc[a], p.loc[b], p.loc[c]
    assert la.strides == lb.strides == (1024, 1) and lc.strides == (1024, 1)
    assert {la.offset, lb.offset} == {lc.offset, lc.offset + 512}
    desc, _ = p._gemm_desc(p.steps[1].nodes[0])
    assert (desc.d_m, desc.d_n) == (1024, 1)


def _epilogue_fn(x, w, h, b):
    y = F.matmul(x, w, "float32", "float32")
    return F.gelu(y) * b + y * h


def _epilogue_fn_keep(x, w, h, b):
    y = F.matmul(x, w, "float32", "float32")
    return F.gelu(y) * b + y * h, y


EPI_SHAPES = [((512, 256), "bfloat16"), ((256, 512), "bfloat16"), ((512, 512), "float32"), ((512,), "float32")]


@pytest.mark.parametrize("fn,keep", [(_epilogue_fn, False), (_epilogue_fn_keep, True)])
def test_elementwise_consumer_of_a_dot_runs_in_its_epilogue(fn, keep, monkeypatch):
    """A loop reading a dot's [m, n] result element for element (with other operands: a broadcast row, a
    same-shape tensor) is merged into the dot: one launch of a generated gemm_epi kernel, which also stores
    the dot's own result when something else (here a graph output) reads it. (The plan fuses only dots with
    enough 256 x 256 tiles to fill the GPU; the threshold is lowered to exercise small shapes.)"""
    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 1)
    with L.config.compiler.patch(horizontal_fusion=False):
        p = _plan(fn, *EPI_SHAPES, build=True)
    assert [s.kind for s in p.steps] == ["dot"]
    st = p.steps[0]
    assert st.epi is not None and st.name.startswith("gemm_epi_") and st.store_dot == keep
    with L.config.compiler.patch(epilogue_fusion=False, horizontal_fusion=False):
        q = _plan(fn, *EPI_SHAPES)
    assert [s.kind for s in q.steps] == ["dot", "loop"]
    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 256)
    with L.config.compiler.patch(horizontal_fusion=False):
        r = _plan(fn, *EPI_SHAPES)
    assert [s.kind for s in r.steps] == ["dot", "loop"]  # 4 tiles: left to the autotuned tiled kernels


def test_large_epilogue_dots_get_their_other_k_loop_for_the_autotuner(monkeypatch):
    """An epilogue GEMM large enough to tune is also generated (and compiled) with the other k loops (k tile 32
    with cross-tile prefetch; k tile 32 with ping-pong waves; k tile 64 on four waves), as separate kernels;
    small ones, or any with the autotuner off, get none."""
    from lumen_amd.compiler import codegen

    monkeypatch.setattr(Plan, "EPI_MIN_TILES", 1)
    monkeypatch.setattr(Plan, "AUTOTUNE_MACS", 1)
    with L.config.compiler.patch(horizontal_fusion=False):
        p = _plan(_epilogue_fn, *EPI_SHAPES, build=True)
    (si, alts), = p.epi_alts.items()
    assert [a[0] for a in alts] == [1, 2, 3, 4]
    for i, (var, k, src) in enumerate(alts):
        bk, kl, wn = codegen.GemmEpilogueKernel.VARIANTS[var]
        assert (bk, kl, wn) == ((32, var, 4) if var < 3 else (64, 3, 2) if var == 3 else (64, 3, 4))
        assert k.name != p.steps[si].name and k.name in src and f", {bk}, {wn}, " in src and f", {kl}>(s, a, b" in src
        assert k.block == (128 * wn, 1, 1) and f"__launch_bounds__({128 * wn})" in src
        assert p.alt_objects[(si, i)].endswith(".hsaco")
    with L.config.compiler.patch(horizontal_fusion=False, autotune=False):
        assert not _plan(_epilogue_fn, *EPI_SHAPES).epi_alts
    monkeypatch.setattr(Plan, "AUTOTUNE_MACS", 1 << 30)
    with L.config.compiler.patch(horizontal_fusion=False):
        assert not _plan(_epilogue_fn, *EPI_SHAPES).epi_alts  # 2^26 multiply-adds


def test_one_row_kernel_for_a_normalization_chain():
    p = _plan(lambda x, w: F.softmax(F.rms_norm(x, 256, w) * 3.0, -1), ((32, 256), "float32"), ((256,), "float32"))
    assert [s.kind for s in p.steps] == ["row"]


@pytest.mark.timeout(600)
def test_generated_kernels_compile_for_gfx950():
    model, opt = W.build(W.TINY)
    ids = L.empty([W.TINY.batch, W.TINY.seq], "int64", "meta")
    p = Plan(trace(W.train_step, (model, opt, ids, ids)).graph, build_kernels=True)
    assert len(p.objects) == len(p.sources) > 10


def test_small_independent_loops_share_one_launch():
    """Horizontal fusion: three small elementwise results that do not read each other become one hloop step
    whose grid is the members' grids end to end; large ones keep their own launches."""
    p = _plan(lambda a, b, c: (a * 2.0, b + 1.0, F.exp(c)), ((64, 64), "float32"), ((128,), "bfloat16"),
              ((1000,), "float32"), build=True)
    kinds = [s.kind for s in p.steps]
    assert kinds.count("hloop") == 1 and "loop" not in kinds
    (si,) = [i for i, s in enumerate(p.steps) if s.kind == "hloop"]
    k = p.kernels[si]
    assert k.grid[0] == sum(m.grid[0] for m in k.parts) and len(k.args) == 6
    big = _plan(lambda a, b: (a * 2.0, b + 1.0), ((2048, 1024), "float32"), ((2048, 1024), "float32"))
    assert [s.kind for s in big.steps] == ["loop", "loop"]


def test_loop_over_a_row_space_joins_the_row_kernel():
    """Softmax statistics (a row kernel) and an elementwise consumer of the same rows reading only the
    row kernel's input, its per-row results and values already in memory: one row kernel writing both."""
    def fn(x, t):
        return L.value_and_grad(lambda x: F.mean(F.cross_entropy(x, t)))(x)

    p = _plan(fn, ((512, 3000), "float32"), ((512,), "int64"))
    big = [s for s in p.steps if s.outputs and p.graph.types[s.outputs[0]].numel() == 512 * 3000
           or any(p.graph.types[v].numel() == 512 * 3000 for v in s.outputs)]
    assert [s.kind for s in big] == ["row"], [(s.kind, s.label()) for s in p.steps]


@pytest.mark.parametrize("v", [32000, 32001])
def test_linear_cross_entropy_is_a_builtin_step_with_bounded_scratch(monkeypatch, v):
    """Primitive::LinearCrossEntropy lowers to one built-in step whose scratch is never the whole [b, v]: with
    bf16 operands, k a multiple of 64 and whole 64-class blocks the fused form's (maximum, sum) pair a row
    and block plus a logit a row; otherwise a chunk of float32 logit rows (Plan.LCE_SCRATCH bytes at most)."""
    from lumen_amd.compiler.plan import Plan
    from lumen_amd.graph import prims

    monkeypatch.setattr(Plan, "LCE_SCRATCH", 1 << 20)
    h = L.empty([4096, 256], "bfloat16", "meta")
    w = L.empty([v, 256], "bfloat16", "meta")
    t = L.empty([4096], "int64", "meta")
    p = Plan(L.make_graph(lambda h, w, t: prims.linear_cross_entropy(h, w, t))(h, w, t), build_kernels=False)
    assert [s.kind for s in p.steps] == ["linear_cross_entropy"]
    d = p._lce_desc(p.steps[0].nodes[0])
    assert d.chunk_rows == (1 << 20) // (v * 4)
    if v % 64 == 0:
        assert p.steps[0].scratch == 4096 * (v // 64) * 8 + 4096 * 4
    else:
        assert p.steps[0].scratch == d.chunk_rows * v * 4


def test_hoisting_casts_into_producers_reads_fewer_bytes(monkeypatch):
    """The config-4 step: the embedding-gradient kernel at the end reads the residual-gradient terms as bf16
    (each cast where its float32 term is made) instead of every float32 term, and the plan's row/loop bytes
    drop against the same plan without the pass."""
    from lumen_amd.compiler import fusion

    cfg = W.CONFIG4
    model, opt = W.build(cfg, lr=1e-2)
    ids = L.empty([cfg.batch, cfg.seq], "int32", "meta")
    tg = L.empty([cfg.batch, cfg.seq], "int32", "meta")
    graph = L.make_graph(W.train_step)(model, opt, ids, tg)

    def loop_bytes(p):
        return sum(p.cost(i)[1] for i, s in enumerate(p.steps) if s.kind in ("loop", "row"))

    with_pass = Plan(graph, build_kernels=False)
    monkeypatch.setattr(fusion, "hoist_to_producers", lambda g, s: s)
    without = Plan(graph, build_kernels=False)
    assert loop_bytes(with_pass) < loop_bytes(without)

    def f32_terms(p):  # float32 [tokens, dim] operands of the row kernel reading the most of them
        g = p.graph
        return max(sum(g.types[v].dtype == "float32" and g.types[v].shape == (cfg.batch * cfg.seq, cfg.dim)
                       for v in s.inputs) for s in p.steps if s.kind == "row")

    assert f32_terms(with_pass) < f32_terms(without)


def test_row_statistics_are_read_only_at_their_own_row():
    """A row kernel holds each statistic for its current row: a broadcast that repeats a row's value over
    its row qualifies, a transposed one (the log-sum-exp of query i spread over the key axis of P^T, as
    grouped-query attention's unfused backward reads it) does not, and fusion keeps such a reader out of
    the row kernel so the generated kernel computes the right values."""
    from lumen_amd.compiler.fusion import row_broadcast
    from lumen_amd.graph.ir import TensorType as T

    rows = (160, 40)
    assert row_broadcast(T("float32", (1, 4, 40, 1)), T("float32", (1, 4, 40, 40)), (0, 1, 2, 3), rows)
    assert row_broadcast(T("float32", (1, 4, 40)), T("float32", (1, 4, 40, 40)), (0, 1, 2), rows)
    assert not row_broadcast(T("float32", (1, 4, 1, 40)), T("float32", (1, 4, 40, 40)), (0, 1, 2, 3), rows)
    assert not row_broadcast(T("float32", (4, 40)), T("float32", (4, 40, 40)), (0, 2), rows)

    rng = np.random.default_rng(0)
    shapes = (1, 40, 4, 32), (1, 40, 2, 32), (1, 40, 2, 32), (1, 40, 4, 32)
    ts = [L.tensor(rng.standard_normal(s).astype(np.float32), "bfloat16") for s in shapes]

    def loss(q, k, v, w):
        return F.sum((F.flash_attention(q, k, v, is_causal=True) * w).float())

    p = Plan(L.make_graph(L.grad(loss, (0, 1, 2)))(*ts), "hip:0", build_kernels=False)
    for si, st in enumerate(p.steps):
        if st.kind == "row":
            assert si in p.sources  # the generated source exists: no statistic read at another row


def _remat_program(x, w, w3, w4):
    a = F.exp(x)                                               # elementwise of an input: cheap to recompute
    h = F.relu(F.matmul(a, w, "float32", "float32"))           # a dot reads it before the peak
    big = F.matmul(h, w3, "float32", "float32")                # the peak: a wide intermediate
    scale = big.sum()                                          # the late dot needs the peak's result ...
    late = F.matmul(a, w4 * scale, "float32", "float32")       # ... and reads `a` again after it
    return late.sum(0)


# `a` and `big` are both 16 MiB: with `a` recomputed, `big` reuses its memory
REMAT_METAS = (((2048, 2048), "float32"), ((2048, 64), "float32"), ((64, 2048), "float32"), ((2048, 64), "float32"))


def test_schedules_keep_the_smallest_workspace():
    """The plan places its steps in the fused order and in the list and depth-first schedules and keeps the
    order needing the least workspace (plan/compile.rs:19-47)."""

    p = _plan(_remat_program, *REMAT_METAS)
    assert set(p.schedule_bytes) == {"fused", "traced", "list", "dfs"}
    assert p.workspace_bytes == min(p.schedule_bytes.values()) or p.schedule == "fused"
    with L.config.compiler.patch(schedules=False):
        q = _plan(_remat_program, *REMAT_METAS)
    assert q.schedule == "fused"


def test_memory_limit_rematerializes_values_without_changing_them():
    """Above ``memory_limit`` a value written before the live-bytes peak and read after it is recomputed
    before its late reader: the workspace shrinks and the oracle computes the same bits from the rewritten
    graph. No schedule helps here: the late dot needs the peak's result."""
    from oracle import oracle

    # horizontal fusion would launch the small recomputation together with the first exp (it groups members
    # of up to 2^20 elements)
    with L.config.compiler.patch(horizontal_fusion=False):
        p0 = _plan(_remat_program, *REMAT_METAS)
        with L.config.compiler.patch(memory_limit=p0.workspace_bytes // 2):
            p1 = _plan(_remat_program, *REMAT_METAS)
    assert p1.workspace_bytes < p0.workspace_bytes
    assert sum(n.prim == "exp" for n in p1.graph.nodes) == 2  # exp(x) computed twice
    rng = np.random.default_rng(0)
    xs = [(rng.standard_normal(s) * 0.1).astype(np.float32) for s, _ in REMAT_METAS]
    for a, b in zip(oracle.run(p0.graph, xs), oracle.run(p1.graph, xs)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _donated(fn, metas, donate):
    g = L.make_graph(fn)(*[L.empty(list(s), d, "meta") for s, d in metas])
    return Plan(g, build_kernels=False, donate=donate)


def test_assigned_weights_of_the_training_step_are_updated_in_place():
    """Each weight the training step assigns is computed over the weight it replaces: its loc is the weight's
    own input, no output copy remains, every step still follows the producers of what it reads, and the
    generated kernels declare the aliased pointers without __restrict__."""
    model, opt = W.build(W.TINY)
    ids = L.empty([W.TINY.batch, W.TINY.seq], "int64", "meta")
    traced = trace(W.train_step, (model, opt, ids, ids))
    at = {k: i for i, (kind, k) in enumerate(traced.layout) if kind == "weight"}
    donate = {traced.n_returned + j: at[k] for j, k in enumerate(traced.written)}
    p = Plan(traced.graph, build_kernels=False, packable=list(at.values()), donate=donate)
    g = p.graph
    assert p.in_place_outputs == donate
    assert not any(st.kind == "copy" for st in p.steps)
    for op, ip in donate.items():
        assert p.output_locs[op].base == ("in", ip) and p.output_locs[op].offset == 0
    made = set(g.inputs)
    for st in p.steps:
        assert all(u in made for u in st.inputs), st.label()
        made.update(st.outputs)
    import re

    checked = 0
    for si, k in p.kernels.items():
        sig = re.search(r"extern \"C\".*?void\s+\w+\((.*?)\)\s*\{", p.sources[si], re.S).group(1).split(", ")
        assert len(sig) == len(k.args), p.sources[si][:300]
        for param, (_, v) in zip(sig, k.args):
            assert ("__restrict__" in param) == (v not in p.aliased), param
            checked += v in p.aliased
    assert checked >= 2 * len(donate)


def test_updates_stay_out_of_place_when_their_input_is_read_elsewhere():
    """An output is not written over its input when its step reads the input at other elements (a transpose)
    or when a step that needs the output still reads the old input; a plain elementwise update is."""
    sq = ((64, 64), "float32")
    p = _donated(lambda w: (w * 0.5,), [sq], {0: 0})
    assert p.in_place_outputs == {0: 0} and p.output_locs[0].base == ("in", 0)
    p = _donated(lambda w: (w - w.t(),), [sq], {0: 0})
    assert p.in_place_outputs == {} and p.output_locs[0].base == ("ws", 0)

    def later(w, x):
        nw = w * 0.5
        return nw, F.matmul(x, nw, "float32", "float32") + F.matmul(x, w, "float32", "float32")

    p = _donated(later, [sq, sq], {0: 0})  # the update moves after the other reader of w
    assert p.in_place_outputs == {0: 0}
    prod = {v: si for si, st in enumerate(p.steps) for v in st.outputs}
    readers = [si for si, st in enumerate(p.steps) if p.graph.inputs[0] in st.inputs]
    assert max(readers) == prod[p.graph.outputs[0]]

    def needed(w, x):
        nw = w * 0.5
        return nw, F.matmul(x, nw, "float32", "float32") + w

    p = _donated(needed, [sq, sq], {0: 0})  # w is read with a result of the update: it cannot move
    assert p.in_place_outputs == {}


def _flash_bwd_steps(b, s, n, d, kvh=None):
    kvh = kvh or n
    metas = [((b, s, n, d), "bfloat16"), ((b, s, kvh, d), "bfloat16"), ((b, s, kvh, d), "bfloat16"),
             ((b, s, n, d), "bfloat16")]

    def loss(q, k, v, w):
        return F.sum((F.flash_attention(q, k, v, is_causal=True) * w).float())

    p = _plan(L.grad(loss, (0, 1, 2)), *metas)
    return [st for st in p.steps if st.kind == "flash_bwd"]


def test_long_sequences_take_the_recomputing_backward_with_o_s_scratch():
    """The deterministic flash backward stores dS (O(Sq x Sk) bytes) only while that fits
    ``attention_ds_max_bytes``; a longer sequence takes the recomputing mode, whose scratch is two floats a
    query row, so the plan's memory grows linearly with the sequence as the reference's backward does."""
    from lumen_amd.compiler import attention as A
    from lumen_amd.config import config

    (short,) = _flash_bwd_steps(1, 1024, 2, 64)
    assert short.mode == 1 and short.scratch >= A.ds_bytes(1, 2, 1024, 1024)
    with config.compiler.patch(attention_ds_max_bytes=1 << 20):
        (long_,) = _flash_bwd_steps(1, 1024, 2, 64)
        assert long_.mode == 2 and long_.scratch == 2 * 1 * 2 * 1024 * 4
        (longer,) = _flash_bwd_steps(1, 4096, 2, 64)
        assert longer.mode == 2 and longer.scratch == 4 * long_.scratch
    with config.compiler.patch(memory_limit=8 * A.ds_bytes(1, 2, 1024, 1024) - 1):
        (limited,) = _flash_bwd_steps(1, 1024, 2, 64)
        assert limited.mode == 2


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("shape", [(1, 1, 1, 1, 64), (2, 3, 200, 333, 128), (1, 4, 4097, 129, 64), (3, 2, 64, 1, 96),
                                   (1, 2, 70, 70, 32)])
def test_flash_backward_scratch_is_what_the_library_reports(mode, shape):
    """The plan sizes a flash backward's scratch by asking the library (nhip_flash_bwd_workspace); checked
    against the layout the kernels write — delta and the LSE (two floats a query row), then, 256-byte
    aligned, the float32 dQ accumulator (mode 0, its head dim padded to the kernel's 64 or 128) or 128 x 64 tiles
    of 16-bit dS (mode 1) — on ragged shapes."""
    from lumen_amd.compiler import attention as A

    b, n, sq, sk, d = shape
    rows = 2 * b * n * sq * 4
    want = {2: rows,
            1: -(-rows // 256) * 256 + b * n * (-(-sk // 128)) * (-(-sq // 64)) * 128 * 64 * 2,
            0: -(-rows // 256) * 256 + b * n * sq * (64 if d <= 64 else 128) * 4}[mode]
    assert A.backward_workspace_bytes(b, n, sq, sk, d, n, mode) == want
    if d == 32 and mode == 0:  # a value head dim above the query's pads the accumulator to the larger one
        assert A.backward_workspace_bytes(b, n, sq, sk, d, n, mode, 96) == want + b * n * sq * 64 * 4


def _chain2(x, a, b):
    t = F.gelu((x * a + b).float())
    return F.softmax(F.layer_norm(t, x.shape[-1]), -1).bfloat16()


def test_gelu_softmax_and_row_divisions_take_their_short_forms():
    """The config-2 chain's row kernel evaluates the traced tanh GELU in its sigmoid form (gelu_tanh_f32, no
    tanh_f32), softmax's exponent of the row-shifted value as one exp2 (exp_shifted_f32) and both row
    divisions as multiplies by the row's reciprocal (fdiv_rowm); exp and division elsewhere keep their
    within-4-ulp and within-1-ulp forms."""
    p = _plan(_chain2, ((64, 512), "bfloat16"), ((512,), "bfloat16"), ((512,), "bfloat16"))
    (src,) = p.sources.values()
    body = src[src.index('extern "C"'):]
    n = body.count("gelu_tanh_f32(")  # one an element a thread
    assert n >= 8 and "tanh_f32(" not in body.replace("gelu_tanh_f32(", "")
    assert body.count("exp_shifted_f32(") == n and "exp_f32(" not in body.replace("exp_shifted_f32(", "")
    assert body.count("fdiv_rowm(") == 2 * n and "fdiv_f32(" not in body and "fdiv_row(" not in body
    q = _plan(lambda x, y: F.exp(x) / y, ((64, 512), "float32"), ((64, 512), "float32"))
    (src,) = q.sources.values()
    body = src[src.index('extern "C"'):]
    assert "exp_f32(" in body and "fdiv_f32(" in body and "exp_shifted_f32(" not in body


def test_one_plus_tanh_keeps_tanh_when_tanh_is_read_elsewhere():
    """1 + tanh(u) becomes 2 sigmoid(2u) only when nothing else reads the tanh (GELU's backward reads it, so
    the training step keeps tanh_f32 there)."""
    p = _plan(lambda u: (1.0 + F.tanh(u)) * 3.0, ((64, 256), "float32"))
    (src,) = p.sources.values()
    body = src[src.index('extern "C"'):]
    assert "onep_tanh_f32(" in body and "tanh_f32(" not in body.replace("onep_tanh", "")
    p = _plan(lambda u: F.tanh(u * 0.5) + 1.0, ((64, 256), "float32"))
    (src,) = p.sources.values()
    body = src[src.index('extern "C"'):]
    assert "onep_tanh_k(" in body and "tanh_f32(" not in body.replace("onep_tanh", "")
    p = _plan(lambda u: (1.0 + F.tanh(u)) * F.tanh(u), ((64, 256), "float32"))
    (src,) = p.sources.values()
    body = src[src.index('extern "C"'):]
    assert "tanh_f32(" in body and "onep_tanh" not in body


def test_training_step_gelu_takes_the_sigmoid_forms():
    """In the training step, the forward GELU (whose tanh the backward recomputes from the stored
    pre-activation) runs in its sigmoid form, and the backward's traced derivative times its cotangent as one
    closed form (gelu_tanh_grad_f32); no kernel keeps a tanh."""
    model, opt = W.build(W.TINY)
    ids = L.empty([W.TINY.batch, W.TINY.seq], "int64", "meta")
    p = Plan(trace(W.train_step, (model, opt, ids, ids)).graph, build_kernels=False)
    bodies = [src[src.index("struct Epi") if "struct Epi" in src else src.index('extern "C"'):]
              for src in p.sources.values()]
    assert sum("gelu_tanh_f32(" in b for b in bodies) >= 2  # one a layer
    assert sum("gelu_tanh_grad_f32(" in b for b in bodies) >= 2
    assert not any("tanh_f32(" in b.replace("gelu_tanh_f32(", "").replace("gelu_tanh_grad_f32(", "")
                   for b in bodies)


def _gelu_grad_forms(fn):
    p = _plan(fn, ((64, 256), "float32"), ((64, 256), "float32"))
    (src,) = p.sources.values()
    return src[src.index('extern "C"'):]


def test_gelu_gradient_short_form_needs_the_whole_derivative():
    """The closed form replaces an expression only when it is dy times GELU's derivative as a function of
    (x, dy): the traced vjp and a hand-written arrangement of the same terms take it (a term added outside the
    derivative stays outside it); the same terms with one coefficient changed, or with a term added among
    them, keep their traced arithmetic and its tanh."""
    c1, c2 = 0.7978845608028654, 0.044715

    def vjp(x, g):
        _, pull = L.vjp(lambda x: F.gelu(x), x)
        return pull(g)[0]

    def by_hand(scale=1.0, inner=0.0, outer=0.0):
        def f(x, g):
            t = F.tanh((x + x * x * x * c2) * c1)
            a = g * (t + 1.0) * 0.5
            if inner:
                a = a + x * g * inner
            d = a + (x * g) * (1.0 - t * t) * (1.0 + x * x * (3.0 * c2)) * (0.5 * c1 * scale)
            return d + x * outer if outer else d
        return f

    for fn in (vjp, by_hand(), by_hand(outer=1e-3)):
        body = _gelu_grad_forms(fn)
        assert "gelu_tanh_grad_f32(" in body and "tanh" not in body.replace("gelu_tanh_grad_f32(", "")
    for fn in (by_hand(scale=1.001), by_hand(inner=1e-3)):
        body = _gelu_grad_forms(fn)
        assert "gelu_tanh_grad_f32(" not in body and "tanh" in body


def test_row_kernel_indices_split_into_row_and_column():
    """A row kernel reading a value at (row, column) through a gather or a broadcast over leading dims indexes it
    by the row (once a row) and the column, not by decomposing r * C + c with 64-bit divisions for every element
    (the training step's embedding row: the token id read once a row, the table row and the position row
    indexed by the column)."""
    import re

    model, opt = W.build(W.TINY)
    ids = L.empty([W.TINY.batch, W.TINY.seq], "int64", "meta")
    p = Plan(trace(W.train_step, (model, opt, ids, ids)).graph, build_kernels=False)
    gathers = [src for si, src in p.sources.items() if p.steps[si].kind == "row" and "gather" in p.steps[si].label()]
    assert gathers
    for src in gathers:
        body = src[src.index('extern "C"'):]
        for ix in re.findall(r"\bin\d+\[([^\]]*)\]", body):
            assert not ("r * " in ix and "/" in ix), ix


def test_norm_statistics_are_read_not_stored_broadcast():
    """The training step's forward norm rows store the per-row statistic ([rows, 1]) and bf16 values only: no
    step writes a float32 [rows, width] broadcast of a row statistic, nor a float32 copy of a stored bf16 value
    that only loop and row kernels read (they recompute those from what is stored)."""
    model, opt = W.build(W.TINY)
    ids = L.empty([W.TINY.batch, W.TINY.seq], "int64", "meta")
    p = Plan(trace(W.train_step, (model, opt, ids, ids)).graph, build_kernels=False)
    g, prod = p.graph, p.graph.producers()
    for st in p.steps:
        if st.kind not in ("loop", "row"):
            continue
        for v in st.outputs:
            n = prod.get(v)
            if n is None or g.types[v].dtype != "float32" or len(g.types[v].shape) < 2:
                continue
            src = g.types[n.inputs[0]] if n.inputs else None
            assert not (n.prim == "broadcast_in_dim" and src is not None and src.numel() * 8 <= g.types[v].numel()), \
                (st.label(), v)
            readers = [s.kind for s in p.steps if v in s.inputs]
            if readers and all(k in ("loop", "row") for k in readers):  # kernels that can recompute it
                assert not (n.prim == "cast" and src is not None and src.dtype == "bfloat16" and n.inputs[0] in
                            {o for s in p.steps for o in s.outputs}), (st.label(), v)
