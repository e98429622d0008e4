"""GPU parity of the operator catalog and the packed projection path.

Every operator runs through the C ABI (libdlhip.so) and is compared bit for
bit with the contract mirror (oracle/contract.c) on identical BF16 inputs:
the reference's own operator shapes and deterministic operands
(tests/gpu/operator_reference.cpp:60-75, 167-314) and the Qwen3-8B shapes.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def up(device, queue, array):
    return device.upload_array(queue, np.ascontiguousarray(array))


def run_op(queue, name, *args):
    from dolittle_amd import _lib
    _lib.call(name, queue.handle, *args)
    queue.drain()


def down(queue, buf, dtype, count):
    return queue.read(buf, dtype, count)


def test_device_is_gfx950(device):
    assert "gfx950" in device.arch
    assert device.compute_units >= 200


@pytest.mark.parametrize("rows,width", [(3, 128), (3, 4096), (40, 128), (2, 12288), (1, 320)])
def test_rms_norm(device, queue, oracle, rows, width):
    x, w = oracle.operand(rows * width, 1), oracle.operand(width, 2)
    bx, bw, by = up(device, queue, x), up(device, queue, w), device.allocate(rows * width * 2)
    run_op(queue, "dl_rms_norm", 1, bx.ptr(), bw.ptr(), by.ptr(), rows, width, C.c_float(1e-6))
    assert np.array_equal(down(queue, by, np.uint16, rows * width), oracle.rms_norm(x, w, rows, width, 1e-6))


@pytest.mark.parametrize("rows,in_w,out_w", [(1, 128, 33), (1, 128, 1025), (9, 128, 33), (9, 128, 1025),
                                             (1, 4096, 4096), (1, 4096, 1024), (1, 12288, 4096), (3, 20, 1025),
                                             (2, 100, 40)])
def test_projection_rowmajor(device, queue, oracle, rows, in_w, out_w):
    rng = np.random.default_rng(rows * 7 + in_w)
    x = oracle.bf16_from_f32(rng.standard_normal(rows * in_w).astype(np.float32))
    w = oracle.bf16_from_f32((0.05 * rng.standard_normal(out_w * in_w)).astype(np.float32))
    bx, bw, by = up(device, queue, x), up(device, queue, w), device.allocate(rows * out_w * 2)
    run_op(queue, "dl_projection", 1, bx.ptr(), bw.ptr(), by.ptr(), rows, in_w, out_w, None)
    assert np.array_equal(down(queue, by, np.uint16, rows * out_w), oracle.projection(x, w, rows, in_w, out_w))


@pytest.mark.parametrize("in_w,out_w", [(4096, 4096), (4096, 1024), (4096, 12288), (12288, 4096), (4096, 16384),
                                        (256, 2048), (512, 64)])
def test_projection_packed(device, queue, oracle, in_w, out_w):
    """The resident packed layout reproduces the reference tree bit for bit."""
    from dolittle_amd import _lib
    rng = np.random.default_rng(in_w + out_w)
    x = oracle.bf16_from_f32(rng.standard_normal(in_w).astype(np.float32))
    w = oracle.bf16_from_f32((0.02 * rng.standard_normal(out_w * in_w)).astype(np.float32))
    bx, bw, by = up(device, queue, x), up(device, queue, w), device.allocate(out_w * 2)
    nbytes = C.c_uint64()
    _lib.call("dl_projection_packed_bytes", out_w, in_w, C.byref(nbytes))
    packed = device.allocate(nbytes.value)
    run_op(queue, "dl_projection_pack", bw.ptr(), packed.ptr(), out_w, in_w)
    run_op(queue, "dl_projection_packed", bx.ptr(), packed.ptr(), by.ptr(), 1, in_w, out_w, None)
    assert np.array_equal(down(queue, by, np.uint16, out_w), oracle.projection(x, w, 1, in_w, out_w))


@pytest.mark.parametrize("first", [0, 1, 511, 4093, 8191])
def test_rotary(device, queue, oracle, first):
    rows, heads, width = 3, 2, 128
    x = oracle.operand(rows * heads * width, 7)
    bx, by = up(device, queue, x), device.allocate(x.nbytes)
    run_op(queue, "dl_rotary", 1, bx.ptr(), by.ptr(), rows, heads, width, first, C.c_double(1e6), None, 0)
    assert np.array_equal(down(queue, by, np.uint16, x.size), oracle.rotary(x, rows, heads, width, first, 1e6))


def test_rotary_device_position_positioned_output(device, queue, oracle):
    rows, heads, width, pos = 1, 8, 128, 700
    x = oracle.operand(rows * heads * width, 3)
    cache = device.allocate((pos + 1) * heads * width * 2)
    bpos = up(device, queue, np.array([pos], np.uint64))
    bx = up(device, queue, x)
    run_op(queue, "dl_rotary", 1, bx.ptr(), cache.ptr(), rows, heads, width, 0, C.c_double(1e6), bpos.ptr(), 1)
    got = down(queue, cache, np.uint16, (pos + 1) * heads * width)[pos * heads * width:]
    assert np.array_equal(got, oracle.rotary(x, rows, heads, width, pos, 1e6))


@pytest.mark.parametrize("rows,first", [(1, 0), (37, 0), (1, 512), (4, 300), (1, 4607)])
def test_attention(device, queue, oracle, rows, first):
    hq, hkv, width = 32, 8, 128
    total = first + rows
    rng = np.random.default_rng(total)
    q = oracle.bf16_from_f32(rng.standard_normal(rows * hq * width).astype(np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(total * hkv * width).astype(np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(total * hkv * width).astype(np.float32))
    bq, bk, bv = up(device, queue, q), up(device, queue, k), up(device, queue, v)
    by = device.allocate(q.nbytes)
    scale = device.allocate(4)
    run_op(queue, "dl_attention_scale", scale.ptr(), width)
    assert down(queue, scale, np.float32, 1)[0] == oracle.lib().orc_attention_scale(width)
    run_op(queue, "dl_attention", 1, bq.ptr(), bk.ptr(), bv.ptr(), by.ptr(), rows, hq, hkv, width, first, None,
           total, scale.ptr())
    assert np.array_equal(down(queue, by, np.uint16, q.size), oracle.attention(q, k, v, rows, hq, hkv, width, first))


def test_attention_reference_operands(device, queue, oracle):
    """operator_reference.cpp:273-313 shapes: 4 heads, 2 KV heads, width 128."""
    for rows in (1, 37):
        q, k, v = oracle.operand(rows * 4 * 128, 8), oracle.operand(rows * 2 * 128, 9), oracle.operand(rows * 2 * 128, 10)
        bq, bk, bv, by = up(device, queue, q), up(device, queue, k), up(device, queue, v), device.allocate(q.nbytes)
        scale = device.allocate(4)
        run_op(queue, "dl_attention_scale", scale.ptr(), 128)
        run_op(queue, "dl_attention", 1, bq.ptr(), bk.ptr(), bv.ptr(), by.ptr(), rows, 4, 2, 128, 0, None, rows,
               scale.ptr())
        assert np.array_equal(down(queue, by, np.uint16, q.size), oracle.attention(q, k, v, rows, 4, 2, 128, 0))


def test_elementwise(device, queue, oracle):
    n = 3 * 259
    x, u = oracle.operand(n, 3), oracle.operand(n, 4)
    x[:3] = oracle.bf16_from_f32(np.array([-80.0, 80.0, 0.0], np.float32))
    bx, bu, by = up(device, queue, x), up(device, queue, u), device.allocate(n * 2)
    run_op(queue, "dl_silu_multiply", 1, bx.ptr(), bu.ptr(), by.ptr(), n)
    assert np.array_equal(down(queue, by, np.uint16, n), oracle.silu_multiply(x, u))
    run_op(queue, "dl_add", 1, bx.ptr(), bu.ptr(), by.ptr(), n)
    assert np.array_equal(down(queue, by, np.uint16, n), oracle.add(x, u))
    rng = np.random.default_rng(1)
    big = oracle.bf16_from_f32((rng.standard_normal(12288) * 4).astype(np.float32))
    big2 = oracle.bf16_from_f32(rng.standard_normal(12288).astype(np.float32))
    bx, bu, by = up(device, queue, big), up(device, queue, big2), device.allocate(big.nbytes)
    run_op(queue, "dl_silu_multiply", 1, bx.ptr(), bu.ptr(), by.ptr(), big.size)
    assert np.array_equal(down(queue, by, np.uint16, big.size), oracle.silu_multiply(big, big2))


def test_embedding_and_gather(device, queue, oracle):
    V, D = 1000, 256
    table = oracle.operand(V * D, 5)
    tokens = np.array([3, 999, 0, 1000, 17], np.uint32)  # 1000 is outside the table
    bt, bw, by = up(device, queue, tokens), up(device, queue, table), device.allocate(len(tokens) * D * 2)
    run_op(queue, "dl_embedding", 1, bt.ptr(), bw.ptr(), by.ptr(), len(tokens), D, V)
    got = down(queue, by, np.uint16, len(tokens) * D).reshape(-1, D)
    tab = table.reshape(V, D)
    for i, t in enumerate(tokens):
        assert np.array_equal(got[i], tab[t] if t < V else np.zeros(D, np.uint16))
    rows = (C.c_uint64 * 2)(1, 4)
    out = device.allocate(2 * D * 2)
    run_op(queue, "dl_gather_rows", by.ptr(), out.ptr(), D * 2, rows, 2)
    g = down(queue, out, np.uint16, 2 * D).reshape(2, D)
    assert np.array_equal(g[0], got[1]) and np.array_equal(g[1], got[4])


def test_invalid_arguments_raise(device, queue):
    from dolittle_amd import InvalidArgument, LengthError, _lib
    buf = device.allocate(1024)
    with pytest.raises(InvalidArgument):
        _lib.call("dl_projection", queue.handle, 3, buf.ptr(), buf.ptr(), buf.ptr(), 1, 4, 4, None)
    with pytest.raises(InvalidArgument):
        _lib.call("dl_attention", queue.handle, 1, buf.ptr(), buf.ptr(), buf.ptr(), buf.ptr(), 1, 3, 2, 128, 0, None,
                  1, buf.ptr())
    with pytest.raises(LengthError):
        _lib.call("dl_projection_pack", queue.handle, buf.ptr(), buf.ptr(), 33, 128)
