"""Host side of the drop-in surface (no GPU): the staged HBM seeds before a
run, arg_names and tensor_input_output_sizes."""
import numpy as np
import pytest

from ktir_cpu_amd import configs
from ktir_cpu_amd.interpreter import KTIRInterpreter
from ktir_cpu_amd.memory import DeviceHBM


def test_staged_hbm_allocate_write_read():
    """Reference memory.py semantics before anything is on the device:
    allocation from 0x10000 in 128-byte sticks, a write to an unmapped
    address makes an allocation there, a write inside one truncates at its
    end, reads zero-pad past the end and raise on unmapped addresses."""
    h = DeviceHBM()
    assert h.allocate(100) == 0x10000 // 128
    assert h.allocate(1) == 0x10000 // 128 + 1
    assert h.allocate(0) == 0x10000 // 128 + 2
    h.write(0, np.arange(8, dtype=np.float16))
    np.testing.assert_array_equal(h.read(0, 10, "f16"), np.array([0, 1, 2, 3, 4, 5, 6, 7, 0, 0], np.float16))
    h.write(0, np.array([9, 9, 9], np.float16), intra_byte=12)           # elements 6.. (truncated at 8)
    np.testing.assert_array_equal(h.read(0, 8, "f16"), np.array([0, 1, 2, 3, 4, 5, 9, 9], np.float16))
    np.testing.assert_array_equal(h.read(0, 3, "f16", intra_byte=4), np.array([2, 3, 4], np.float16))
    np.testing.assert_array_equal(h.read(0, 0, "f16", offsets=np.array([1, 7, 50])),
                                  np.array([1, 9, 0], np.float16))
    with pytest.raises(ValueError):
        h.read(5, 1, "f16")
    with pytest.raises(ValueError):
        h.write(5, np.zeros(2, np.float16), offsets=np.array([0, 1]))
    assert [a for a, _ in h.staged()] == [0]


def test_prepare_execution_gives_fresh_memory():
    interp = KTIRInterpreter()
    interp.load(configs.vector_add(4096, 128, 32))
    interp._prepare_execution((32, 1, 1))
    m1 = interp.memory
    assert m1.num_cores == 32 and m1.hbm.next_ptr == 0x10000
    interp._prepare_execution((32, 1, 1))
    assert interp.memory is not m1


def test_arg_names_and_sizes_of_every_config():
    """Names in declaration order; sizes from the first memory view of each
    pointer (reference ir_types.py:565-573)."""
    cases = [
        (configs.vector_add(4096, 128, 32), "add_kernel", ["x_ptr", "y_ptr", "output_ptr", "BLOCK_SIZE"],
         {"x_ptr": ((4096,), "f16"), "y_ptr": ((4096,), "f16"), "output_ptr": ((4096,), "f16")}),
        (configs.gather_scatter_add(1024, 32, 512, 4, 32), "gather_scatter_add", ["table_ptr", "idx_ptr", "out_ptr"],
         {"table_ptr": ((1024, 32), "f16"), "idx_ptr": ((512,), "i32"), "out_ptr": ((1024, 32), "f32")}),
        (configs.softmax(64, 256, 8, 4), "softmax_kernel", ["x_ptr", "y_ptr"],
         {"x_ptr": ((64, 256), "f16"), "y_ptr": ((64, 256), "f16")}),
        (configs.rmsnorm(64, 256, 8, 4), "rmsnorm_kernel", ["x_ptr", "w_ptr", "y_ptr", "eps"],
         {"x_ptr": ((64, 256), "f16"), "w_ptr": ((256,), "f16"), "y_ptr": ((64, 256), "f16")}),
        (configs.gemm(256, 256, 256, 64, 64, 32, 2, 2), "gemm_kernel", ["a_ptr", "b_ptr", "c_ptr"],
         {"a_ptr": ((256, 256), "f16"), "b_ptr": ((256, 256), "f16"), "c_ptr": ((256, 256), "f16")}),
    ]
    for src, fn, names, sizes in cases:
        interp = KTIRInterpreter()
        with pytest.raises(RuntimeError):
            interp.arg_names(fn)
        interp.load(src)
        assert interp.arg_names(fn) == names
        got = interp.tensor_input_output_sizes(fn)
        assert {k: (v["shape"], v["dtype"]) for k, v in got.items()} == sizes
        with pytest.raises(ValueError):
            interp.tensor_input_output_sizes("no_such_function")


def test_sizes_key_on_the_first_view_of_a_pointer():
    """A pointer viewed twice keeps its first view's shape."""
    v1 = configs._view("a", "p", [8, 16], [16, 1], "f16")
    v2 = configs._view("b", "p", [128], [1], "f16")
    src = ("module {\n  func.func @k(%p: index) attributes {grid = [1, 1]} {\n"
           + v1 + "\n" + v2 + "\n    return\n  }\n}\n")
    interp = KTIRInterpreter()
    interp.load(src)
    assert interp.tensor_input_output_sizes("k") == {"p": {"shape": (8, 16), "dtype": "f16"}}
