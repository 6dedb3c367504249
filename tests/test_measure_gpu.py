"""The streaming-read measurement kernel (ulspec_stream_read) that the read
ceiling is taken from: every variant (4 .. 32 loads per thread, plain and
non-temporal) reads every 16-byte unit of the buffer once, including a
ragged tail past the last full workgroup, and bad arguments are refused.

A unit is shown to be read by planting the sink's key word in it alone: the
thread that loads it XORs its units to the key and writes the sink, which no
other thread does (all other units are zero).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

KEY = 0x5EED5EED


def _read(ctx, units, plant, variant):
    buf = np.zeros((units, 4), np.uint32)
    if plant is not None:
        buf[plant, 0] = KEY
    b = ctx.upload(buf)
    sink = ctx.upload(np.zeros(4, np.uint32))
    ctx.stream_read(b, units * 16, variant, sink)
    ctx.sync()
    out = int(ctx.download(sink, np.uint32, (4,))[0])
    b.free()
    sink.free()
    return out


@pytest.mark.parametrize("variant", range(8))
def test_stream_read_reads_every_unit(ctx, variant):
    U = 4 << (variant & 3)
    units = 3 * 256 * U + 77  # three full workgroups and a ragged fourth
    for plant in (0, 255, 256 * U - 1, 256 * U, 2 * 256 * U + 13, units - 1):
        assert _read(ctx, units, plant, variant) == KEY, f"unit {plant} not read"
    assert _read(ctx, units, None, variant) == 0


def test_stream_read_argument_errors(ctx, pkg):
    b = ctx.alloc(64)
    sink = ctx.alloc(16)
    for nbytes, variant in ((0, 0), (24, 0), (64, 8)):
        with pytest.raises(pkg.UlspecError) as e:
            ctx.stream_read(b, nbytes, variant, sink)
        assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        ctx.stream_read(b, 64, 0, None)
    assert e.value.status == pkg.EINVAL
    b.free()
    sink.free()
