"""The device C-ABI (include/ferrograd_hip.h), ported from the reference's
backend tests (src/device/cpu.rs:415-649, src/device.rs:366-477) to HIP:
compile-and-launch of hand-written kernels and the forceable error paths."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ADD = r"""
extern "C" __global__ void add(const float* a, const float* b, float* out, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i];
}"""

MUL = r"""
extern "C" __global__ void mul(float* out, const float* a, const float* b) {
  int i = threadIdx.x;
  if (i < 3) out[i] = a[i] * b[i];
}"""

NEG = r"""
extern "C" __global__ void negate(float* output, const float* input) {
  int i = threadIdx.x;
  if (i < 3) output[i] = -input[i];
}"""

MIXED = r"""
extern "C" __global__ void add_offset(float* out, const float* input, int offset, float scale) {
  int i = threadIdx.x;
  if (i < 2) out[i] = (input[offset + i] * scale);
}"""

SCALE_BOOL = r"""
extern "C" __global__ void scale(const float* data, float* out, int n, float scalar, bool flip) {
  int i = threadIdx.x;
  if (i < n) out[i] = flip ? -data[i] * scalar : data[i] * scalar;
}"""


@pytest.fixture(scope="module")
def ctx(fg):
    from ferrograd_amd.hip import Context

    return Context(0)


def _upload(ctx, arr):
    p = ctx.alloc(arr.nbytes)
    ctx.h2d(p, arr)
    return p


def _download(ctx, p, n, dtype=np.float32):
    out = np.empty(n, dtype=dtype)
    ctx.d2h(out, p)
    return out


def test_device_info_is_gfx950(ctx):
    info = ctx.info()
    assert info["arch"].startswith("gfx950"), info
    assert info["cu_count"] >= 256


def test_compile_and_launch_add(ctx):  # cpu.rs:415-436
    from ferrograd_amd.hip import Arg

    prog = ctx.compile(ADD, "add", 4)
    a = _upload(ctx, np.array([1, 2, 3], np.float32))
    b = _upload(ctx, np.array([4, 5, 6], np.float32))
    o = ctx.alloc(12)
    ctx.launch(prog, [Arg.ptr(a), Arg.ptr(b), Arg.ptr(o), Arg.i32(3)], grid=(1, 1, 1), block=(64, 1, 1))
    assert _download(ctx, o, 3).tolist() == [5.0, 7.0, 9.0]


def test_device_mul_output_slot0(ctx):  # cpu.rs:559-583
    from ferrograd_amd.hip import Arg

    prog = ctx.compile(MUL, "mul", 3)
    o = ctx.alloc(12)
    a = _upload(ctx, np.array([2, 3, 4], np.float32))
    b = _upload(ctx, np.array([5, 6, 7], np.float32))
    ctx.launch(prog, [Arg.ptr(o), Arg.ptr(a), Arg.ptr(b)])
    assert _download(ctx, o, 3).tolist() == [10.0, 18.0, 28.0]


def test_device_unary(ctx):  # cpu.rs:585-608
    from ferrograd_amd.hip import Arg

    prog = ctx.compile(NEG, "negate", 2)
    o = ctx.alloc(12)
    i = _upload(ctx, np.array([1, -2, 3], np.float32))
    ctx.launch(prog, [Arg.ptr(o), Arg.ptr(i)])
    assert _download(ctx, o, 3).tolist() == [-1.0, 2.0, -3.0]


def test_device_mixed_scalar_args(ctx):  # cpu.rs:610-637
    from ferrograd_amd.hip import Arg

    prog = ctx.compile(MIXED, "add_offset", 4)
    o = ctx.alloc(8)
    i = _upload(ctx, np.array([1, 2, 3, 4], np.float32))
    ctx.launch(prog, [Arg.ptr(o), Arg.ptr(i), Arg.i32(1), Arg.f32(10.0)])
    assert _download(ctx, o, 2).tolist() == [20.0, 30.0]


def test_scalar_and_bool_args(ctx):  # cpu.rs:461-482 plus the u8 bool ABI (cpu.rs:108-113)
    from ferrograd_amd.hip import Arg

    prog = ctx.compile(SCALE_BOOL, "scale", 5)
    d = _upload(ctx, np.array([1, 2, 3, 4], np.float32))
    o = ctx.alloc(16)
    ctx.launch(prog, [Arg.ptr(d), Arg.ptr(o), Arg.i32(4), Arg.f32(3.0), Arg.boolean(False)])
    assert _download(ctx, o, 4).tolist() == [3.0, 6.0, 9.0, 12.0]
    ctx.launch(prog, [Arg.ptr(d), Arg.ptr(o), Arg.i32(4), Arg.f32(3.0), Arg.boolean(True)])
    assert _download(ctx, o, 4).tolist() == [-3.0, -6.0, -9.0, -12.0]


def test_alloc_is_zeroed(ctx):  # device.rs:366-377, cpu.rs:277-280
    p = ctx.alloc(4096, zero=True)
    assert not _download(ctx, p, 1024).any()
    ctx.free(p)
    q = ctx.alloc(4096, zero=True)  # a reused block is zeroed again
    assert not _download(ctx, q, 1024).any()


@pytest.mark.parametrize("nbytes", [4, (1 << 20) - 4, 1 << 20, (1 << 20) + 4, 3 << 20, (4 << 20) - 4, 4 << 20,
                                    (5 << 20) + 4, (16 << 20) + 4, (40 << 20) + 12])
def test_copies_round_trip_on_both_sides_of_the_staging_limits(ctx, nbytes):
    # Host->device copies up to 64 KiB go through a pinned staging ring and
    # device->host reads up to 1 MiB land in a pinned buffer; from 4 MiB both
    # go through two pinned 16 MiB chunks in turn (partial last chunk
    # included); the sizes between go direct. Every size must round-trip
    # exactly.
    n = nbytes // 4
    a = np.random.default_rng(nbytes).standard_normal(n).astype(np.float32)
    p = _upload(ctx, a)
    assert np.array_equal(_download(ctx, p, n), a)
    ctx.free(p)


def test_chunked_copies_back_to_back(ctx):
    # Three uploads through the pinned chunks queued without a wait between
    # them (each refills a chunk only once its previous DMA has finished),
    # then the reads, each against its source.
    sizes = [(24 << 20) + 8, (5 << 20) + 4, 33 << 20]
    arrays = [np.random.default_rng(i).standard_normal(n // 4).astype(np.float32) for i, n in enumerate(sizes)]
    ptrs = [_upload(ctx, a) for a in arrays]
    for p, a in zip(ptrs, arrays):
        assert np.array_equal(_download(ctx, p, a.size), a)
        ctx.free(p)


def test_chunked_copies_from_two_threads(ctx):
    # Two contexts used on two threads at once: both copy through the host
    # copy pool (one job at a time) and get their own bytes back.
    import threading

    from ferrograd_amd.hip import Context

    ctx2 = Context(0)
    arrays = [np.random.default_rng(10 + i).standard_normal((12 << 20) // 4 + i).astype(np.float32) for i in range(2)]
    got, errors = [None, None], []

    def run(i, c):
        try:
            for _ in range(3):
                p = _upload(c, arrays[i])
                got[i] = _download(c, p, arrays[i].size)
                c.free(p)
        except Exception as e:  # reported below, on the test's thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i, c)) for i, c in enumerate((ctx, ctx2))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        assert np.array_equal(got[i], arrays[i])


def test_bad_source_is_compile_error(ctx):  # cpu.rs:484-497, 639-649
    from ferrograd_amd.hip import FG_ERR_COMPILE, HipError

    with pytest.raises(HipError) as e:
        ctx.compile("this is not valid HIP!", "nope", 1)
    assert e.value.code == FG_ERR_COMPILE
    assert "hiprtc compilation failed" in str(e.value)


def test_wrong_symbol_is_symbol_error(ctx):  # cpu.rs:499-516
    from ferrograd_amd.hip import FG_ERR_SYMBOL, HipError

    src = 'extern "C" __global__ void real_name(float* a, int n) {}'
    with pytest.raises(HipError) as e:
        ctx.compile(src, "wrong_name", 2)
    assert e.value.code == FG_ERR_SYMBOL


def test_wrong_arg_count_is_rejected(ctx):  # cpu.rs:331-336
    from ferrograd_amd.hip import FG_ERR_ARGS, Arg, HipError

    prog = ctx.compile(NEG, "negate", 2)
    o = ctx.alloc(12)
    with pytest.raises(HipError) as e:
        ctx.launch(prog, [Arg.ptr(o)])
    assert e.value.code == FG_ERR_ARGS
    assert "expected 2 kernel args, got 1" in str(e.value)


def test_events_time_kernels(ctx):
    from ferrograd_amd.hip import Arg

    prog = ctx.compile(ADD, "add", 4)
    n = 1 << 20
    a = ctx.alloc(4 * n)
    b = ctx.alloc(4 * n)
    o = ctx.alloc(4 * n)
    ctx.record(0)
    ctx.launch(prog, [Arg.ptr(a), Arg.ptr(b), Arg.ptr(o), Arg.i32(n)], grid=(n // 256, 1, 1), block=(256, 1, 1))
    ctx.record(1)
    assert ctx.elapsed_ms(0, 1) > 0.0


# ── HIP-graph replay and allocator hints (no counterpart in the reference) ──

AXPY = r"""
extern "C" __global__ void axpy(float* y, const float* x, float a, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = y[i] * a + x[i];
}"""


def test_graph_replays_launches_in_order_with_updated_arguments(ctx):
    from ferrograd_amd.hip import Arg

    n = 1000
    prog = ctx.compile(AXPY, "axpy", 4)
    x1 = _upload(ctx, np.arange(n, dtype=np.float32))
    x2 = _upload(ctx, np.full(n, 2.0, np.float32))
    ya = _upload(ctx, np.ones(n, np.float32))
    yb = _upload(ctx, np.zeros(n, np.float32))
    grid, block = ((n + 255) // 256, 1, 1), (256, 1, 1)
    # y = (y * 3 + x1) * 0.5 + x2: two dependent launches, order matters.
    seq = lambda y, a: [(prog, [Arg.ptr(y), Arg.ptr(x1), Arg.f32(a), Arg.i32(n)], grid, block, 0),  # noqa: E731
                        (prog, [Arg.ptr(y), Arg.ptr(x2), Arg.f32(0.5), Arg.i32(n)], grid, block, 0)]
    g = ctx.graph_create(seq(ya, 3.0))  # records only: nothing runs
    assert np.array_equal(_download(ctx, ya, n), np.ones(n, np.float32))
    flat = lambda s: [a for l in s for a in l[1]]  # noqa: E731
    assert ctx.graph_launch(g, flat(seq(ya, 3.0))) == 0
    want = (np.ones(n, np.float32) * 3 + np.arange(n, dtype=np.float32)) * np.float32(0.5) + 2
    assert np.array_equal(_download(ctx, ya, n), want.astype(np.float32))
    # Another buffer and scalar: the first launch is updated, the second too (y).
    assert ctx.graph_launch(g, flat(seq(yb, -1.0))) == 2
    want_b = (np.zeros(n, np.float32) * -1 + np.arange(n, dtype=np.float32)) * np.float32(0.5) + 2
    assert np.array_equal(_download(ctx, yb, n), want_b.astype(np.float32))
    assert np.array_equal(_download(ctx, ya, n), want.astype(np.float32))  # untouched
    ctx.graph_free(g)


def test_graph_create_rejects_a_wrong_argument_count(ctx):
    from ferrograd_amd.hip import Arg, HipError

    prog = ctx.compile(AXPY, "axpy", 4)
    y = ctx.alloc(16)
    with pytest.raises(HipError, match="wrong argument count"):
        ctx.graph_create([(prog, [Arg.ptr(y), Arg.f32(1.0)], (1, 1, 1), (64, 1, 1), 0)])


def test_alloc_hint_returns_the_hinted_free_block(ctx):
    a, b = ctx.alloc(1 << 20, zero=False), ctx.alloc(1 << 20, zero=False)
    ctx.free(a)
    ctx.free(b)  # the LIFO free list would hand out b first
    assert ctx.alloc_hint(1 << 20, a) == a
    assert ctx.alloc_hint(1 << 20, 0) == b
    ctx.free(a)
    ctx.free(b)
    c = ctx.alloc_hint(1 << 21, a)  # another size: the hint does not apply
    assert c not in (a, b)
    ctx.free(c)


@pytest.mark.gpu
def test_hip_device_copy_from_host_size_error(fg, hip):  # device.rs:457-466, cpu.rs:294-300
    # The HIP device's own size check (the reference's message), reached
    # through Device::copy_from_host on a realised tensor's buffer.
    t = fg.Tensor.new(np.ones(2, np.float32), [2], hip)
    with pytest.raises(fg.FerrogradError, match="copy_from_host: expected 8 bytes, got 4"):
        t.write(np.ones(1, np.float32))
    t.write(np.array([3.0, 4.0], np.float32))
    assert t.to_vec() == [3.0, 4.0]
    z = fg.Tensor.zeros([3], hip)  # lazily zero-filled storage is materialised first
    z.write(np.array([1.0, 2.0, 3.0], np.float32))
    assert z.to_vec() == [1.0, 2.0, 3.0]
