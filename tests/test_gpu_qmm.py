"""Parity of the HIP quantised matmul (hb_qmm / rs_mlx_op 3,10x) with the CPU
oracle (oracle.qmm, pinned to native/projection_reference.h)."""
import numpy as np
import pytest

import oracle
from numerics import assert_bf16_close, assert_close

pytestmark = pytest.mark.gpu


def run_qmm(hb, x_bits, packed, scales, biases, M, N, K, group=64, bits=4, y_f32=False):
    from hip_bridge import DeviceBuffer, LAYOUT_MLX, LAYOUT_Q4T

    dx = DeviceBuffer.from_array(x_bits)
    dw = DeviceBuffer.from_array(packed)
    ds = DeviceBuffer.from_array(scales)
    db = DeviceBuffer.from_array(biases)
    dy = DeviceBuffer(M * N * (4 if y_f32 else 2))
    layout = LAYOUT_MLX
    if bits == 4 and group == 64 and N % 16 == 0 and K % 128 == 0:
        dwt, dsb = DeviceBuffer(packed.nbytes), DeviceBuffer(scales.nbytes * 2)
        hb.q4_tile(dw, ds, db, dwt, dsb, N, K)
        dw, ds, db, layout = dwt, dsb, None, LAYOUT_Q4T
    hb.qmm(dx, dw, ds, db, dy, M, N, K, group, bits, layout, y_f32)
    hb.synchronize()
    if y_f32:
        return dy.download(np.float32, (M, N))
    return hb.quant.bf16_value(dy.download(np.uint16, (M, N)))


def reference(x_bits, packed, scales, biases, group=64, bits=4):
    from hip_bridge import quant

    return oracle.qmm(quant.bf16_value(x_bits), packed, quant.bf16_value(scales), quant.bf16_value(biases), group,
                      bits)


@pytest.fixture(scope="module")
def hb(bridge):
    import hip_bridge.quant  # noqa: F401

    return bridge


def test_qgemv_config_shape(hb):
    # x bf16 [8, 2048], W [6144, 2048] 4-bit g64, y bf16 [8, 6144]
    x, packed, s, b = hb.quant.qgemv_workload()
    print("case: qgemv 8x6144x2048 seed 20261201", flush=True)
    y = run_qmm(hb, x, packed, s, b, 8, 6144, 2048)
    assert_bf16_close(y, reference(x, packed, s, b), "qgemv 8x6144x2048")


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (3, 96, 128), (5, 112, 256), (8, 48, 2048), (16, 512, 512),
                                   (17, 256, 1024), (32, 128, 2048), (40, 192, 512), (64, 64, 4096),
                                   (256, 96, 2048), (2, 100, 192), (7, 33, 64)])
def test_qmm_shapes(hb, M, N, K):
    x, packed, s, b = hb.quant.qgemv_workload(M, N, K, seed=M * 1000 + N)
    print(f"case: qmm M={M} N={N} K={K}", flush=True)
    for y_f32 in (False, True):
        y = run_qmm(hb, x, packed, s, b, M, N, K, y_f32=y_f32)
        assert_bf16_close(y, reference(x, packed, s, b), f"qmm {M}x{N}x{K} f32={y_f32}")


@pytest.mark.parametrize("M,N,K", [(17, 256, 1024), (64, 512, 2048), (128, 768, 4096), (256, 256, 256),
                                   (33, 1024, 512), (200, 512, 4096)])
def test_qmm_streaming_tiles(hb, M, N, K):
    """M > 16 with 256-row weight groups: the persistent streaming kernel (one
    pass for K <= 2048, f32 passes over 2048-wide column blocks above), in all
    three output modes, with an output row stride wider than N."""
    from hip_bridge import DeviceBuffer, LAYOUT_Q4T

    x, packed, s, b = hb.quant.qgemv_workload(M, N, K, seed=M * 7 + K)
    want = reference(x, packed, s, b)
    ldy = N + 32
    dx, dw, ds, db = (DeviceBuffer.from_array(a) for a in (x, packed, s, b))
    dwt, dsb = DeviceBuffer(packed.nbytes), DeviceBuffer(s.nbytes * 2)
    hb.q4_tile(dw, ds, db, dwt, dsb, N, K)
    print(f"case: streaming qmm M={M} N={N} K={K}", flush=True)
    init = np.random.default_rng(K).standard_normal((M, ldy)).astype(np.float32)
    for mode in (0, 1, 2):
        dy = DeviceBuffer.from_array(init) if mode == 2 else DeviceBuffer(M * ldy * 4)
        hb.qmm(dx, dwt, dsb, None, dy, M, N, K, 64, 4, LAYOUT_Q4T, ldy=ldy, out_mode=mode)
        hb.synchronize()
        if mode == 0:
            got = hb.quant.bf16_value(dy.download(np.uint16, (M, ldy)))[:, :N]
            assert_bf16_close(got, want, f"bf16 out {M}x{N}x{K}")
        else:
            got = dy.download(np.float32, (M, ldy))
            base = init if mode == 2 else 0.0
            assert_bf16_close(got[:, :N] - (base[:, :N] if mode == 2 else 0.0), want, f"mode {mode} {M}x{N}x{K}")
            if mode == 2:
                assert np.array_equal(got[:, N:], init[:, N:]), "columns past N untouched"


@pytest.mark.parametrize("M,N,K", [(128, 10240, 2048), (100, 12544, 2048), (250, 9216, 1024), (48, 40960, 1024)])
def test_qmm_two_tile_projection(hb, M, N, K):
    """M > 16 with enough 256-row groups x 32-token pairs to fill the GPU: the
    projection kernel that holds a token pair's x in LDS and runs each
    dequantized weight fragment against both token tiles, streaming a range of
    weight groups per workgroup, in all three output modes with an output row
    stride wider than N; ragged M, one and two 1024-column chunks, one and
    several groups per workgroup; two runs agree bit for bit."""
    from hip_bridge import DeviceBuffer, LAYOUT_Q4T

    x, packed, s, b = hb.quant.qgemv_workload(M, N, K, seed=M + N + K)
    want = reference(x, packed, s, b)
    ldy = N + 32
    dx, dw, ds, db = (DeviceBuffer.from_array(a) for a in (x, packed, s, b))
    dwt, dsb = DeviceBuffer(packed.nbytes), DeviceBuffer(s.nbytes * 2)
    hb.q4_tile(dw, ds, db, dwt, dsb, N, K)
    print(f"case: two-tile projection M={M} N={N} K={K}", flush=True)
    init = np.random.default_rng(K).standard_normal((M, ldy)).astype(np.float32)
    for mode in (0, 1, 2):
        dy = DeviceBuffer.from_array(init) if mode == 2 else DeviceBuffer(M * ldy * 4)
        hb.qmm(dx, dwt, dsb, None, dy, M, N, K, 64, 4, LAYOUT_Q4T, ldy=ldy, out_mode=mode)
        hb.synchronize()
        if mode == 0:
            got = hb.quant.bf16_value(dy.download(np.uint16, (M, ldy)))[:, :N]
        else:
            got = dy.download(np.float32, (M, ldy))
            if mode == 2:
                assert np.array_equal(got[:, N:], init[:, N:]), "columns past N untouched"
                got = got - init
            got = got[:, :N]
        assert_bf16_close(got, want, f"two-tile projection {M}x{N}x{K} mode {mode}")
        if mode == 1:
            again = DeviceBuffer(M * ldy * 4)
            hb.qmm(dx, dwt, dsb, None, again, M, N, K, 64, 4, LAYOUT_Q4T, ldy=ldy, out_mode=1)
            hb.synchronize()
            assert np.array_equal(again.download(np.float32, (M, ldy))[:, :N], got), "run to run"


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_qmm_generic_bits(hb, bits, group):
    M, N, K = 5, 40, group * 4
    x, packed, s, b = hb.quant.qgemv_workload(M, N, K, group, bits, seed=bits * 7 + group)
    print(f"case: generic qmm bits={bits} group={group}", flush=True)
    y = run_qmm(hb, x, packed, s, b, M, N, K, group, bits, y_f32=True)
    assert_close(y, reference(x, packed, s, b, group, bits), 1e-5, f"generic bits={bits} group={group}")


def test_graph_api_all_ones(hb):
    # tests/native_execution.rs:103-128 through rs_mlx_input/op/finish
    from hip_bridge import GraphHandle

    for bits in [2, 3, 4, 5, 6, 8]:
        for group in [32, 64, 128]:
            g = GraphHandle(1)
            x = g.input(np.ones((2, group), np.float32))
            w = g.input(np.full((3, group * bits // 32), 0xFFFFFFFF, np.uint32))
            s = g.input(np.full((3, 1), 0.125, np.float32))
            b = g.input(np.full((3, 1), -0.25, np.float32))
            y = g.op(100 + bits, [x, w, s, b], group)
            out = g.finish(y, (2, 3))
            assert np.allclose(out, group * (((1 << bits) - 1) * 0.125 - 0.25), rtol=1e-6), (bits, group, out)


def test_graph_api_mixed_bitstream(hb):
    # tests/native_execution.rs:286-322
    from hip_bridge import GraphHandle

    for bits in [2, 3, 4, 5, 6, 8]:
        for group in [32, 64, 128]:
            k = group * 2
            packed = np.zeros(3 * k * bits // 32, np.uint64)
            x = np.array([((j % 11) - 5) / 8 for j in range(2 * k)], np.float32)
            expected = np.zeros(6)
            for row in range(3):
                for j in range(k):
                    q = (j * 7 + row * 3) % (1 << bits)
                    bit = (row * k + j) * bits
                    word, shift = bit // 32, bit % 32
                    packed[word] |= (q << shift) & 0xFFFFFFFF
                    if shift + bits > 32:
                        packed[word + 1] |= q >> (32 - shift)
                    for bb in range(2):
                        expected[bb * 3 + row] += float(x[bb * k + j]) * (q * 0.125 - 0.25)
            g = GraphHandle(1)
            xi = g.input(x.reshape(2, k))
            wi = g.input(packed.astype(np.uint32).reshape(3, -1))
            si = g.input(np.full((3, 2), 0.125, np.float32))
            bi = g.input(np.full((3, 2), -0.25, np.float32))
            y = g.op(100 + bits, [xi, wi, si, bi], group)
            out = g.finish(y, (2, 3))
            assert np.allclose(out.reshape(-1), expected, rtol=1e-5, atol=1e-5), (bits, group)


def test_graph_api_rejections(hb):
    from hip_bridge import GraphHandle, HipBridgeError

    g = GraphHandle(1)
    x = g.input(np.ones((2, 64), np.float32))
    w = g.input(np.zeros((3, 8), np.uint32))
    s = g.input(np.ones((3, 1), np.float32))
    with pytest.raises(HipBridgeError, match="invalid operand count"):
        g.op(104, [x, w, s], 64)
    with pytest.raises(HipBridgeError, match="invalid node reference"):
        g.op(104, [x, w, s, 99], 64)
    with pytest.raises(HipBridgeError, match="unsupported affine quantization"):
        g.op(104, [x, w, s, s], 48)
    with pytest.raises(HipBridgeError, match="output size mismatch"):
        g.finish(x, (3, 3))


@pytest.mark.parametrize("M,N,K,vocab", [(256, 16384, 2048, 16000), (100, 32768, 2048, 32768), (64, 16384, 2048, 9000),
                                         (64, 16384, 1024, 9000), (128, 152064, 2048, 151936),
                                         (256, 152064, 2048, 151936)])
def test_fused_head_selection(hb, M, N, K, vocab):
    """Greedy selection fused into the vocabulary-head projection (no logits
    written) against the projection's own f32 logits run through the two-level
    argmax: identical winners, margins (bit for bit) and non-finite status.
    Planted: duplicated weight rows (exact ties: lowest index, margin 0), a tie
    across the vocab limit (the padding row must not count), and one token row
    of x with a huge value (a non-finite logit sets only that row's status)."""
    import ctypes as C

    from hip_bridge import LAYOUT_Q4T, DeviceBuffer, call, load

    x, packed, s, b = hb.quant.qgemv_workload(M, N, K, seed=M * 3 + N + K)
    boost = lambda v: ((v.astype(np.uint32) << 16).view(np.float32) * np.float32(64)).view(np.uint32) >> 16
    for r in (5000, 3):  # rows that win for about half the tokens
        s[r], b[r] = boost(s[r]).astype(np.uint16), boost(b[r]).astype(np.uint16)
    for dst, src in ((7, 5000), (N - 256 - 3, 11), (vocab, 3)):  # ties; the last sits past vocab
        if dst < N:
            packed[dst], s[dst], b[dst] = packed[src], s[src], b[src]
    x[M // 2, :] = 0x7F7F  # bf16 3.39e38 on every column: the row's logits overflow
    dx, dw, ds, db = (DeviceBuffer.from_array(a) for a in (x, packed, s, b))
    dwt, dsb = DeviceBuffer(packed.nbytes), DeviceBuffer(s.nbytes * 2)
    hb.q4_tile(dw, ds, db, dwt, dsb, N, K)
    print(f"case: fused head selection M={M} N={N} K={K} vocab={vocab}", flush=True)
    dy = DeviceBuffer(M * N * 4)
    hb.qmm(dx, dwt, dsb, None, dy, M, N, K, 64, 4, LAYOUT_Q4T, ldy=N, out_mode=1)
    ws = DeviceBuffer(int(load().hb_argmax_workspace_bytes(M, vocab)))
    want = [DeviceBuffer(M * 4) for _ in range(3)]
    call("hb_argmax_margin", dy, N, M, vocab, *want, ws, None)
    pws = DeviceBuffer(int(load().hb_qmm_select_workspace_bytes(M, N)))
    got = [DeviceBuffer(M * 4) for _ in range(3)]
    fused = C.c_int(-1)
    call("hb_qmm_select", dx, M, K, dwt, dsb, N, vocab, pws, pws.nbytes, *got, C.byref(fused), None)
    hb.synchronize()
    if K != 2048:
        assert fused.value == 0, "only K = 2048 (the vocabulary head's hidden size) is fused"
        return
    assert fused.value == 1, "the shape runs the fused kernel"
    wg, wm, st = (d.download(t, (M,)) for d, t in zip(got, (np.uint32, np.float32, np.int32)))
    ww, wmm, wst = (d.download(t, (M,)) for d, t in zip(want, (np.uint32, np.float32, np.int32)))
    ok = wst == 0
    assert np.array_equal(st, wst) and wst[M // 2] == 1 and ok.sum() == M - 1, "non-finite status"
    assert np.array_equal(wg[ok], ww[ok]), "winners"
    assert np.array_equal(wm[ok].view(np.uint32), wmm[ok].view(np.uint32)), "margins"
    logits = dy.download(np.float32, (M, N))[ok]
    assert (wg[ok] < vocab).all() and (wg[ok] != 5000).all(), "padding rows and the later twin never win"
    tie = wg[ok] == 7
    assert tie.any() and (wm[ok][tie] == 0).all(), "the duplicated row wins some tokens with margin 0"
    top = np.argmax(logits[:, :vocab], axis=1)
    assert np.array_equal(top.astype(np.uint32), wg[ok]), "numpy argmax (first maximum) of the same logits"
    if N == 152064:
        # the vocabulary head's own shape (hidden 2048, vocab 151936 in 152064
        # tiled rows): the logits of a few tokens against the FP64 oracle, and
        # the fused winner against the oracle's winner where its margin is
        # clear of the observed logit error
        sel = [0, 1, M // 2 - 1, M // 2 + 1, M - 1]
        want_l = oracle.qmm(hb.quant.bf16_value(x[sel]), packed, hb.quant.bf16_value(s), hb.quant.bf16_value(b), 64, 4)
        got_l = dy.download(np.float32, (M, N))[sel]
        assert_close(got_l[:, :vocab], want_l[:, :vocab], 1e-3, "vocabulary-head logits at 152064 x 2048")
        for j, t in enumerate(sel):
            ow, om = oracle.winner(want_l[j, :vocab].astype(np.float32))
            err = float(np.max(np.abs(got_l[j, :vocab] - want_l[j, :vocab])))
            if om > 2 * err:
                assert wg[t] == ow, f"token {t}: fused winner {wg[t]} != oracle winner {ow}"


@pytest.mark.parametrize("N,K,mode", [(12544, 2048, 0), (9216, 2048, 0), (2048, 4096, 2), (2048, 4096, 1),
                                      (768, 2048, 1), (152064, 2048, 1), (2048, 1024, 2)])
def test_rows_do_not_depend_on_the_batch(hb, N, K, mode):
    """Every dense matmul shape of the decoder (DeltaNet and attention
    in-projections, the K = 4096 output projections accumulating into the
    residual, the MTP fc, the router, the vocabulary head, a K = 1024 case) gives
    bitwise-identical rows whatever the number of packed tokens above 16: the
    first M rows of one input at M = 17, 64, 128 and 256. Greedy decoding with
    speculation then emits the same stream as decoding one token per row."""
    from hip_bridge import DeviceBuffer

    rng = np.random.default_rng(N + K + mode)
    _, packed, s, b = hb.quant.qgemv_workload(16, N, K, seed=N + K)
    tw = hb.TiledWeight(packed, s, b)
    x = hb.quant.bf16_bits(rng.standard_normal((256, K), dtype=np.float32))
    res0 = rng.standard_normal((256, N)).astype(np.float32)
    outs = {}
    for M in (256, 128, 64, 17):
        print(f"case: batch invariance N={N} K={K} mode={mode} M={M}", flush=True)
        dx = DeviceBuffer.from_array(np.ascontiguousarray(x[:M]))
        dy = DeviceBuffer.from_array(np.ascontiguousarray(res0[:M])) if mode == 2 else DeviceBuffer(
            M * N * (2 if mode == 0 else 4))
        hb.qmm(dx, tw.w, tw.sb, None, dy, M, N, K, out_mode=mode)
        hb.synchronize()
        outs[M] = dy.download(np.uint16 if mode == 0 else np.uint32, (M, N))
    for M in (128, 64, 17):
        diff = int(np.sum(outs[M] != outs[256][:M]))
        assert diff == 0, f"M={M}: {diff} outputs differ from the same rows at M=256"


def _tree_group_sums(h_bits):
    """Group sums of bf16 rows in the fixed order of the producers and the
    projections: per 8 columns (((lo0 + hi0) + (lo1 + hi1)) + ...) from zero in
    f32, then the 8 partials of a 64-column group as ((p0 + p1) + (p2 + p3)) +
    ((p4 + p5) + (p6 + p7))."""
    v = (h_bits.astype(np.uint32) << 16).view(np.float32)
    M, K = v.shape
    q = v.reshape(M, K // 8, 4, 2)
    part = np.zeros((M, K // 8), np.float32)
    for k in range(4):
        part = (part + (q[:, :, k, 0] + q[:, :, k, 1])).astype(np.float32)
    p = part.reshape(M, K // 64, 8)
    a = ((p[..., 0] + p[..., 1]) + (p[..., 2] + p[..., 3])).astype(np.float32)
    b = ((p[..., 4] + p[..., 5]) + (p[..., 6] + p[..., 7])).astype(np.float32)
    return (a + b).astype(np.float32)


@pytest.mark.parametrize("N", [12544, 9216])
@pytest.mark.parametrize("M", [17, 64, 100, 128, 200, 256])
def test_projection_with_producer_group_sums(hb, M, N):
    """The input norm writing the group sums of its bf16 rows (hb_rmsnorm_gs)
    and the in-projection reading them (hb_qmm_gs) give the same bits as
    hb_rmsnorm + hb_qmm; the sums themselves match a numpy restatement of the
    fixed order bit for bit."""
    from hip_bridge import DeviceBuffer

    K = 2048
    rng = np.random.default_rng(M * 7 + N)
    _, packed, s, b = hb.quant.qgemv_workload(16, N, K, seed=M + N)
    tw = hb.TiledWeight(packed, s, b)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 20.0, (M, 1))).astype(np.float32)
    w = (1 + 0.3 * rng.standard_normal(K)).astype(np.float32)
    dx, dw = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
    print(f"case: producer group sums M={M} N={N}", flush=True)
    h0, h1, gs = DeviceBuffer(M * K * 2), DeviceBuffer(M * K * 2), DeviceBuffer(M * (K // 64) * 4)
    hb.call("hb_rmsnorm", dx, K, dw, M, K, 1e-6, h0, K, None, None)
    hb.call("hb_rmsnorm_gs", dx, K, dw, M, K, 1e-6, h1, K, gs, None)
    y0, y1 = DeviceBuffer(M * N * 2), DeviceBuffer(M * N * 2)
    hb.qmm(h0, tw.w, tw.sb, None, y0, M, N, K, out_mode=0)
    hb.call("hb_qmm_gs", h1, tw.w, tw.sb, y1, M, N, K, 0, N, gs, None)
    hb.synchronize()
    hbits = h0.download(np.uint16, (M, K))
    assert np.array_equal(hbits, h1.download(np.uint16, (M, K))), "normalised rows"
    want = _tree_group_sums(hbits)
    got = gs.download(np.float32, (M, K // 64))
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), "group sums"
    a, c = y0.download(np.uint16, (M, N)), y1.download(np.uint16, (M, N))
    assert np.array_equal(a, c), f"projection: {int(np.sum(a != c))} outputs differ"
