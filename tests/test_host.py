"""CPU-only checks of the device library: it loads, exports every symbol the
C header declares, and its host-side planning (the pairwise-tree layout every
bit-exact kernel uses, the split-K plan) agrees with the oracle and the
reference's rules. No device calls."""
from __future__ import annotations

import ctypes
import re
from ctypes import byref, c_int64, c_uint32
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from conftest import ROOT
from vkml_amd import _lib

HEADER = ROOT / "include" / "vkhip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vkhip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in vkhip.h but not exported: {missing}"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with vkhip.h"


def test_calls_before_init_fail_cleanly():
    lib = _lib.load()
    if lib.vkhip_get_stream():
        pytest.skip("backend already initialised in this process")
    code = lib.vkhip_synchronize()
    assert code == _lib.ERR_NOT_INITIALISED
    assert b"not initialised" in lib.vkhip_last_error()


def leaf_layout(n: int):
    lib = _lib.load()
    d, b, e = c_uint32(), c_uint32(), c_uint32()
    assert lib.vkhip_pairwise_leaf(n, 0, byref(d), byref(b), byref(e)) == 0
    leaves = []
    for j in range(1 << d.value):
        assert lib.vkhip_pairwise_leaf(n, j, None, byref(b), byref(e)) == 0
        leaves.append((b.value, e.value))
    return d.value, leaves


def carry_fold(vals) -> np.float32:
    stack, count = {}, 0
    for v in vals:
        block, c, level = np.float32(v), count, 0
        while c & 1:
            block = np.float32(block + stack[level])
            c >>= 1
            level += 1
        stack[level] = block
        count += 1
    total, level = np.float32(0.0), 0
    while (count >> level) != 0:
        if (count >> level) & 1:
            total = np.float32(total + stack[level])
        level += 1
    return total


@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 48, 64, 65, 100, 127, 784, 1000, 1023, 1025,
                               4096, 4097, 9999, 32768, 100003])
def test_device_tree_layout_reproduces_the_oracle_sum(n):
    """The device kernels sum each depth-D leaf sequentially and combine the
    2^D leaf values adjacent-first (a balanced fold). Done here on the CPU with
    the library's own leaf table, that must equal the oracle bit for bit."""
    depth, leaves = leaf_layout(n)
    # leaves tile [0, n) in order; non-leftmost descendants are empty
    covered = [i for b, e in leaves for i in range(b, e)]
    assert covered == list(range(n))
    assert all(e - b <= 32 for b, e in leaves)
    rng = np.random.default_rng(n)
    for scale in (1.0, 1e4):
        v = (rng.standard_normal(n) * scale).astype(np.float32)
        v[::7] *= np.float32(1e3)
        sums = []
        for b, e in leaves:
            sums.append(np.float32(0.0) if e == b else np.cumsum(v[b:e], dtype=np.float32)[-1])
        got = carry_fold(sums) if sums else np.float32(0.0)
        assert got.tobytes() == O.pairwise_sum(v).tobytes(), (n, depth)


def plan(batch, m, n, k, split=0):
    lib = _lib.load()
    s, c = c_uint32(), c_uint32()
    assert lib.vkhip_gemm_plan(batch, m, n, k, split, byref(s), byref(c)) == 0
    return s.value, c.value


def test_split_k_plan_rules():
    """The split-K plan: equal chunks of K-tiles, workspace <= 64 MiB, OFF
    never splits, a forced request gets the largest power-of-two chunk giving
    at least that many partitions (reference plan_split_k,
    vulkan_backend.cpp:596-647); AUTO splits K in two when 64x64 tiles are
    exactly one round of one workgroup per CU, and otherwise exactly when
    neither 128x128 nor 64x64 output tiles give each of the 256 CUs a
    workgroup, and then takes as
    many partitions as fit one round of one workgroup per CU (the rule
    restated for MI355X)."""
    # the GEMM sweep's square sizes down to 2048^3 and 8192x1024x4096 fill the
    # machine with 128x128 or 64x64 tiles: no split
    assert plan(1, 4096, 4096, 4096) == (1, 128)
    assert plan(1, 8192, 1024, 4096)[0] == 1
    assert plan(1, 2048, 2048, 2048)[0] == 1
    # exactly one round of 64x64 tiles with K >= 16 K-tiles: two partitions
    # (run as the two halves of one workgroup); fewer K-tiles, or batches,
    # stay unsplit
    assert plan(1, 1024, 1024, 1024) == (2, 16)
    assert plan(1, 1024, 1024, 1056) == (2, 17)
    assert plan(1, 1024, 1024, 480)[0] == 1
    assert plan(2, 1024, 512, 1024)[0] == 1
    # 512^3: 64 tiles of 64x64 -> four partitions of four K-tiles
    assert plan(1, 512, 512, 512) == (4, 4)
    # the skinny K-dominant BASELINE shapes and the small MLP/conv GEMMs split
    for m, n, k in [(256, 256, 65536), (128, 784, 16384), (64, 128, 784), (128, 1024, 576)]:
        splits, chunk = plan(1, m, n, k)
        ktiles = -(-k // 32)
        assert splits > 1 and chunk >= 2
        assert splits == -(-ktiles // chunk)
        assert m * n * splits * 4 <= 64 << 20
        tiles = -(-m // 64) * -(-n // 64)
        assert tiles * splits >= min(512, tiles * (ktiles // 2)) // 2
    # one round of 256 workgroups, then twice the partitions for pairs (two K
    # streams per workgroup) when each keeps >= 8 K-tiles and the pairs still
    # fit one round: 4 tiles x 64 -> 128 partitions of 16 K-tiles (64 pairs
    # per tile); unless 128x64 tiles, three workgroups per CU, promise less
    # matrix-core time: 13 such tiles x 57 partitions of 9 K-tiles for
    # 128x784x16384 (784 columns pad to 832 instead of 896)
    assert plan(1, 256, 256, 65536) == (128, 16)
    assert plan(1, 128, 784, 16384) == (57, 9)
    # partitions below 8 K-tiles are not paired: 8 tiles of 128x64 x 86
    # partitions of 6 against 4 tiles x 64 unpaired partitions of 8
    assert plan(1, 256, 256, 16384) == (86, 6)
    # K of 4 K-tiles or fewer is never split (the fold would cost more)
    assert plan(1, 64, 10, 128)[0] == 1 and plan(1, 128, 256, 100)[0] == 1
    assert plan(1, 128, 100, 256)[0] > 1
    # more than half a round of tiles (144 at 1536^3): power-of-two chunk
    assert plan(1, 1536, 1536, 1536) == (3, 16)
    # a batched conv GEMM has tiles enough
    assert plan(128, 128, 1024, 576)[0] == 1
    # OFF
    assert plan(1, 256, 256, 65536, split=1)[0] == 1
    # forced request: chunk is the largest power of two giving >= request splits
    s, c = plan(1, 64, 64, 4096, split=8)
    assert c == 16 and s == 8


def test_unfold_and_operand_helpers():
    d = _lib.operand((3, 5), (5, 1))
    assert list(d.ne) == [1, 1, 3, 5] and list(d.nb) == [0, 0, 5, 1]
    u = _lib.unfold((3, 2), (1, 2), (1, 0), (1, 1), (7, 5))
    assert (u.kernel_h, u.kernel_w, u.stride_w, u.pad_h, u.image_h) == (3, 2, 2, 1, 7)


def test_fast_divide_is_exact():
    """The launch-time division the movement kernels use, against Python's //,
    over small, large, boundary and random numerators and divisors."""
    lib = _lib.load()
    rng = np.random.default_rng(0)
    divisors = [1, 2, 3, 5, 7, 9, 16, 17, 31, 32, 33, 100, 1000, 1024, 4095, 65535, 65536,
                (1 << 31) - 1, 1 << 31, (1 << 31) + 1, (1 << 32) - 1]
    divisors += [int(d) for d in rng.integers(1, 1 << 32, 40, dtype=np.uint64)]
    for d in divisors:
        nums = [0, 1, d - 1, d, d + 1, 2 * d - 1, (1 << 32) - 1, (1 << 32) - 2, (1 << 31)]
        nums += [int(v) for v in rng.integers(0, 1 << 32, 200, dtype=np.uint64)]
        for n in nums:
            n &= 0xFFFFFFFF
            assert lib.vkhip_fast_divide(n, d) == n // d, (n, d)


@pytest.mark.parametrize("shape,kernel,stride,pad,dil", [
    ((1, 1, 4, 4), (2, 2), (1, 1), (0, 0), (1, 1)),
    ((1, 3, 5, 5), (3, 3), (1, 1), (1, 1), (1, 1)),
    ((1, 2, 6, 6), (2, 2), (2, 2), (0, 0), (1, 1)),
    ((1, 1, 7, 5), (3, 2), (2, 1), (1, 0), (1, 1)),
    ((1, 2, 5, 5), (2, 2), (1, 1), (0, 0), (2, 2)),
    ((1, 3, 9, 11), (5, 3), (2, 3), (2, 1), (1, 2)),
])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
@pytest.mark.parametrize("gather", ["vkhip_im2col_offset", "vkhip_im2col_offset_t"])
def test_implicit_im2col_map_matches_the_oracle_unfold(shape, kernel, stride, pad, dil, layout, gather):
    """The (row, pos) -> image offset maps the convolution GEMMs gather with
    (the forward's register-path loader; the weight gradient's LDS-direct
    loader), evaluated by the library's own host build of the device
    functions, pick exactly the oracle's im2col element for every column
    entry (0 where the window covers padding), for a plain and a channels-last
    image layout."""
    lib = _lib.load()
    offset_of = getattr(lib, gather)
    _, c, h, w = shape
    img = np.arange(c * h * w, dtype=np.float32).reshape(c, h, w) + 1.0
    strides = (h * w, w, 1) if layout == "nchw" else (1, w * c, c)
    storage = np.zeros(c * h * w, np.float32)
    for ci in range(c):
        for y in range(h):
            for xx in range(w):
                storage[ci * strides[0] + y * strides[1] + xx * strides[2]] = img[ci, y, xx]
    want = O.im2col(img[None], kernel, stride, pad, dil)[0]
    u = _lib.unfold(kernel, stride, pad, dil, (h, w))
    st = (c_int64 * 3)(*strides)
    off = c_int64()
    got = np.empty_like(want)
    for row in range(want.shape[0]):
        for pos in range(want.shape[1]):
            assert offset_of(byref(u), c, st, row, pos, byref(off)) == 0
            got[row, pos] = 0.0 if off.value < 0 else storage[off.value]
    assert got.tobytes() == want.tobytes()


def _kcd_stage_accesses(lib, rows_tile, s_row, row0, rows, k0, kdim):
    """Every (LDS float index, byte offset) a KCD stage of `rows_tile` rows
    loads, from the library's host build of the loader's slot map."""
    out = []
    for slot in range(rows_tile * 8):
        off = lib.vkhip_kcd_slot_offset(slot, s_row, row0, rows, k0, kdim)
        out.append((4 * slot, None if off & 0x80000000 else off))
    return out


@pytest.mark.parametrize("cout,k", [(4, 27), (64, 27), (2, 18), (6, 45), (64, 576), (128, 1152),
                                    (5, 8), (128, 784)])
def test_kcd_loader_stays_inside_the_operand_when_its_conditions_hold(cout, k):
    """The straight-to-LDS (KCD) loader's accesses for a [Cout, K] weight
    operand, replayed on the host from the library's own slot map over every
    K-tile and row tile: each 16-byte stage slot is written once, inside the
    stage. With K a multiple of four (the condition the kernels launch it
    under) every load is 16-byte aligned and inside the operand. With K not a
    multiple of four -- the convolution weights' A operand of CIFAR conv1 and
    of the first conv test geometry, K = 3*3*3 = 27 -- loads start at
    addresses that are not 16-byte aligned and the last row's last group
    reads past the operand's end: what a conv kernel loading its weights this
    way did before it ended in a GPU memory fault, and why conv2d_forward only
    takes the straight-to-LDS paths when K % 4 == 0."""
    lib = _lib.load()
    nbytes = cout * k * 4
    misaligned = overrun = 0
    for rows_tile in (64, 128):
        for row0 in range(0, cout, rows_tile):
            for k0 in range(0, k, 32):
                acc = _kcd_stage_accesses(lib, rows_tile, k, row0, cout, k0, k)
                assert sorted(i for i, _ in acc) == list(range(0, rows_tile * 32, 4))
                for _, off in acc:
                    if off is None:
                        continue
                    misaligned += off % 16 != 0
                    overrun += off + 16 > nbytes
    if k % 4 == 0:
        assert misaligned == 0 and overrun == 0
    else:
        assert misaligned > 0 and overrun > 0


# ---- node extent checks (vkhip_supports is host-only: no device needed) ----

def _tensor(shape, dtype=_lib.F32, strides=None, data=0x1000):
    t = _lib.TensorDesc()
    t.data = data
    t.dtype = dtype
    t.ndim = len(shape)
    if strides is None:
        strides, s = [], 1
        for e in reversed(shape):
            strides.insert(0, s)
            s *= e
    for i, (e, st) in enumerate(zip(shape, strides)):
        t.ne[i] = e
        t.nb[i] = st
    return t


def _node(op, out, srcs, params=b""):
    nd = _lib.NodeDesc()
    nd.op = _lib.OP[op]
    nd.n_src = len(srcs)
    nd.out = out
    for i, s in enumerate(srcs):
        nd.src[i] = s
    for i, b in enumerate(params):
        nd.params[i] = b
    return nd


def _unfold_bytes(k, s, p, d, hw):
    u = _lib.unfold((k, k), (s, s), (p, p), (d, d), hw)
    return bytes(u)


def _mask(*axes):
    return int(sum(1 << a for a in axes)).to_bytes(4, "little")


# (name, well-formed node, malformed variants): every malformed node must be
# refused before any launch, because the kernels size their reads and writes
# from params and the operands, not from the output tensor.
def _extent_cases():
    conv = _unfold_bytes(3, 1, 1, 1, (8, 8))
    return [
        ("matmul", _node("MATMUL", _tensor((4, 5)), [_tensor((4, 3)), _tensor((3, 5))]),
         [_node("MATMUL", _tensor((4, 6)), [_tensor((4, 3)), _tensor((3, 5))]),
          _node("MATMUL", _tensor((5, 5)), [_tensor((4, 3)), _tensor((3, 5))]),
          _node("MATMUL", _tensor((4, 5)), [_tensor((4, 3)), _tensor((2, 5))]),
          _node("MATMUL", _tensor((2, 4, 5)), [_tensor((3, 4, 3)), _tensor((3, 5))]),
          _node("MATMUL", _tensor((3, 4, 5)), [_tensor((2, 4, 3)), _tensor((3, 3, 5))])]),
        ("matmul_batch", _node("MATMUL", _tensor((2, 3, 4, 5)),
                               [_tensor((2, 1, 4, 3)), _tensor((1, 3, 3, 5))]), []),
        ("softmax", _node("SOFTMAX", _tensor((6, 7)), [_tensor((6, 7))], (1).to_bytes(4, "little")),
         [_node("SOFTMAX", _tensor((6, 8)), [_tensor((6, 7))], (1).to_bytes(4, "little")),
          _node("LOG_SOFTMAX", _tensor((42,)), [_tensor((6, 7))], (1).to_bytes(4, "little"))]),
        ("sum", _node("SUM", _tensor((6,)), [_tensor((6, 7))], _mask(1)),
         [_node("SUM", _tensor((7,)), [_tensor((6, 7))], _mask(1)),
          _node("SUM", _tensor((6,)), [_tensor((6, 7))], _mask(1, 2))]),
        ("argmax", _node("ARGMAX", _tensor((7,), _lib.I64), [_tensor((6, 7))], _mask(0)),
         [_node("ARGMAX", _tensor((6,), _lib.I64), [_tensor((6, 7))], _mask(0))]),
        ("im2col", _node("IM2COL", _tensor((2, 27, 64)), [_tensor((2, 3, 8, 8))], conv),
         [_node("IM2COL", _tensor((2, 27, 63)), [_tensor((2, 3, 8, 8))], conv),
          _node("IM2COL", _tensor((2, 26, 64)), [_tensor((2, 3, 8, 8))], conv),
          _node("IM2COL", _tensor((1, 27, 64)), [_tensor((2, 3, 8, 8))], conv),
          _node("IM2COL", _tensor((2, 27, 64)), [_tensor((2, 3, 8, 9))], conv)]),
        ("col2im", _node("COL2IM", _tensor((2, 3, 8, 8)), [_tensor((2, 27, 64))], conv),
         [_node("COL2IM", _tensor((2, 3, 8, 7)), [_tensor((2, 27, 64))], conv),
          _node("COL2IM", _tensor((2, 4, 8, 8)), [_tensor((2, 27, 64))], conv),
          _node("COL2IM", _tensor((2, 3, 8, 8)), [_tensor((2, 27, 60))], conv),
          _node("COL2IM", _tensor((3, 3, 8, 8)), [_tensor((2, 27, 64))], conv)]),
        ("max_pool2d", _node("MAX_POOL2D", _tensor((2, 3, 4, 4)), [_tensor((2, 3, 8, 8))],
                             _unfold_bytes(2, 2, 0, 1, (8, 8))),
         [_node("MAX_POOL2D", _tensor((2, 3, 4, 5)), [_tensor((2, 3, 8, 8))],
                _unfold_bytes(2, 2, 0, 1, (8, 8))),
          _node("MAX_POOL2D", _tensor((2, 3, 4, 4)), [_tensor((2, 3, 8, 9))],
                _unfold_bytes(2, 2, 0, 1, (8, 8)))]),
        ("max_pool2d_backward", _node("MAX_POOL2D_BACKWARD", _tensor((2, 3, 8, 8)),
                                      [_tensor((2, 3, 4, 4)), _tensor((2, 3, 8, 8))],
                                      _unfold_bytes(2, 2, 0, 1, (8, 8))),
         [_node("MAX_POOL2D_BACKWARD", _tensor((2, 3, 8, 8)),
                [_tensor((2, 3, 4, 3)), _tensor((2, 3, 8, 8))], _unfold_bytes(2, 2, 0, 1, (8, 8))),
          _node("MAX_POOL2D_BACKWARD", _tensor((2, 3, 8, 4)),
                [_tensor((2, 3, 4, 4)), _tensor((2, 3, 8, 8))], _unfold_bytes(2, 2, 0, 1, (8, 8)))]),
    ]


@pytest.mark.parametrize("case", _extent_cases(), ids=lambda c: c[0])
def test_supports_refuses_nodes_whose_extents_disagree(case):
    """A node whose output (or col2im source) extents disagree with what its
    params and operands imply is not supported, so compute() refuses it with
    VKHIP_ERR_INVALID before any launch instead of writing out of bounds."""
    from ctypes import byref as ref

    lib = _lib.load()
    name, good, bad = case
    assert lib.vkhip_supports(ref(good)) == 1, (name, lib.vkhip_last_error())
    for i, nd in enumerate(bad):
        assert lib.vkhip_supports(ref(nd)) == 0, f"{name}: malformed variant {i} accepted"


def _vec_node(op, out_addr, srcs, n=64):
    """A node record over fake device addresses: f32 vectors of n elements
    (the planner compares byte spans and never dereferences them)."""
    nd = _lib.NodeDesc()
    nd.op = op

    def desc(t, addr):
        t.data = addr
        t.dtype = 0
        t.ndim = 1
        t.ne[0] = n
        t.nb[0] = 1

    desc(nd.out, out_addr)
    nd.n_src = len(srcs)
    for i, a in enumerate(srcs):
        desc(nd.src[i], a)
    return nd


def _output_order(nodes, outputs):
    lib = _lib.load()
    arr = (_lib.NodeDesc * len(nodes))(*nodes)
    outs = (_lib.Copy * len(outputs))(*[_lib.Copy(None, a, n) for a, n in outputs])
    order = (ctypes.c_size_t * len(nodes))()
    after = ctypes.c_size_t()
    assert lib.vkhip_program_output_order(arr, len(nodes), outs, len(outputs), order,
                                          ctypes.byref(after)) == 0
    return list(order), after.value


def test_program_output_order_hoists_the_output_cone_within_hazards():
    """vkhip_program_set_outputs' reordering, on node records over fake
    addresses: the units the output depends on (a loss row node and its mean)
    move ahead of later-recorded units they share no bytes with, keep their own
    order, and stop behind the writer of what they read; a unit that writes
    bytes they read (WAR), reads bytes they write (RAW the other way) or writes
    the same bytes (WAW) is not passed. `after` counts the units that run before
    the outputs are final."""
    B = 1 << 20  # spans of 256 bytes, far apart
    X, LOGITS, G1, G2, ROWS, LOSS, W, OTHER = (B * (i + 1) for i in range(8))
    fwd = _vec_node(54, LOGITS, [X, W])          # logits = f(x, w)
    bwd1 = _vec_node(97, G1, [LOGITS, X])        # gradient chain reads logits
    bwd2 = _vec_node(54, G2, [G1, X])
    upd = _vec_node(17, W, [W, G2])              # the update writes w
    rows = _vec_node(96, ROWS, [LOGITS, X])      # the loss rows
    mean = _vec_node(48, LOSS, [ROWS])           # the output
    order, after = _output_order([fwd, bwd1, bwd2, upd, rows, mean], [(LOSS, 4)])
    assert order == [0, 4, 5, 1, 2, 3] and after == 3

    # The update overwrites the logits' buffer (a WAR hazard for the loss rows): no move.
    upd_war = _vec_node(17, LOGITS, [LOGITS, G2])
    order, after = _output_order([fwd, bwd1, bwd2, upd_war, rows, mean], [(LOSS, 4)])
    assert order == [0, 1, 2, 3, 4, 5] and after == 6

    # A unit reading the bytes the loss rows write (they hold an older value
    # there) keeps the rows behind it; the mean stays behind the rows.
    reader = _vec_node(54, OTHER, [ROWS, X])
    order, after = _output_order([fwd, bwd1, reader, bwd2, rows, mean], [(LOSS, 4)])
    assert order == [0, 1, 2, 4, 5, 3] and after == 5

    # A unit writing part of the bytes the loss rows write (WAW), where the
    # mean reads only the other part (so that unit stays out of the cone), is
    # not passed either.
    half = _vec_node(54, ROWS + 128, [G1, X], n=32)
    mean32 = _vec_node(48, LOSS, [ROWS], n=32)
    order, after = _output_order([fwd, bwd1, half, bwd2, rows, mean32], [(LOSS, 4)])
    assert order == [0, 1, 2, 4, 5, 3] and after == 5

    # Another writer of the output's bytes joins the cone: the cone keeps its
    # order, so the output is final behind the last writer.
    seed = _vec_node(2, LOSS, [])
    order, after = _output_order([fwd, bwd1, seed, bwd2, rows, mean], [(LOSS, 4)])
    assert order == [0, 2, 4, 5, 1, 3] and after == 4

    # An output nothing writes is final before the first unit.
    order, after = _output_order([fwd, bwd1], [(OTHER, 4)])
    assert order == [0, 1] and after == 0
