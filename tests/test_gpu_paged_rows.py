"""PagedKV's row accessors (split, rows, rows_of_heads, write_rows) on the kernels, against the
connector's torch indexing restated in oracle/cpu_path.py (core/everserve/state/kvcopy.py:74-128),
byte for byte, in every layout, on and off the 16-byte path, bf16 and fp8."""

import numpy as np
import pytest
import torch

from everserve_amd.state.paged import PagedKV
from oracle import cpu_path
from tests.cases import LAYOUTS, bits, caches

pytestmark = pytest.mark.gpu

SLOTS = [5, 17, 0, 27, 3, 26]
HEADS = [2, 0]


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("d", [8, 6])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_the_row_accessors_read_and_write_what_torch_indexing_does(ext, layout, d, dtype):
    cpu = caches(layout, d, dtype, n_layers=1, seed=81)[0]
    gpu = cpu.cuda()
    paged = PagedKV.of(gpu)
    slots = torch.tensor(SLOTS, dtype=torch.long)
    heads = torch.tensor(HEADS, dtype=torch.long)
    # the ids may come from the host or the device, as int32 or int64
    got = paged.rows_of_heads(gpu, slots.cuda(), heads.int())
    want = cpu_path.rows_of_heads(cpu, slots, heads)
    assert tuple(got.shape) == tuple(want.shape)
    assert np.array_equal(bits(got), bits(want.contiguous()))
    got1 = paged.rows(gpu, slots.int(), 1)
    assert np.array_equal(bits(got1), bits(cpu_path.rows(cpu, slots, 1).contiguous()))
    b, o = paged.split(slots.cuda())
    assert b.cpu().tolist() == [s // paged.block_size for s in SLOTS]
    assert o.cpu().tolist() == [s % paged.block_size for s in SLOTS]
    # write K and V rows of another cache's head into head slot 1
    x = caches(layout, d, dtype, n_layers=1, seed=82)[0]
    x = cpu_path.rows(x, slots, 0).contiguous()
    cpu_path.write_rows(cpu, slots, 1, x)
    paged.write_rows(gpu, slots.cuda(), 1, x.cuda())
    torch.cuda.synchronize()
    assert np.array_equal(bits(gpu), bits(cpu))


def test_write_rows_refuses_rows_of_another_shape_or_dtype(ext):
    gpu = caches("kv_first", 8, torch.bfloat16, n_layers=1, seed=83)[0].cuda()
    paged = PagedKV.of(gpu)
    slots = torch.tensor(SLOTS, dtype=torch.long, device="cuda")
    with pytest.raises(ValueError, match="shape"):
        paged.write_rows(gpu, slots, 0, torch.zeros(2, len(SLOTS) + 1, 8, dtype=torch.bfloat16,
                                                     device="cuda"))
    with pytest.raises(ValueError, match="dtype"):
        paged.write_rows(gpu, slots, 0, torch.zeros(2, len(SLOTS), 8, dtype=torch.float16,
                                                     device="cuda"))
