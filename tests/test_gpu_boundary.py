"""The drop-in surface callers use around execute_function, on the GPU:

* seeding HBM at literal sticks from a wrapped ``_prepare_execution(grid)``
  and reading it back through ``interp.memory.hbm`` (the reference's pattern,
  ``tests/test_indirect_access.py:122-155``, golden Y = [[12, 9, 6, 3]] x 4);
* ``arg_names`` / ``tensor_input_output_sizes`` driving the inputs
  (``tests/test_examples.py:149-166``).
"""
import numpy as np
import pytest

from ktir_cpu_amd import configs
from tests import _cases

pytestmark = pytest.mark.gpu


def _gather_4x4_literal():
    """Y[m, k] = X[IDX1[m, k], IDX2[m, k]] with every tensor at a literal
    element address: X f16 at element 0 (stick 0), IDX1 i32 at element 32
    (stick 1), IDX2 i32 at element 64 (stick 2), Y f16 at element 192 (stick 3)."""
    cs = "affine_set<(d0, d1) : (d0 >= 0, -d0 + 3 >= 0, d1 >= 0, -d1 + 3 >= 0)>"
    views = "\n".join(configs._view(v, a, [4, 4], [4, 1], dt) for v, a, dt in
                      (("xv", "xa", "f16"), ("i1v", "i1a", "i32"), ("i2v", "i2a", "i32"), ("yv", "ya", "f16")))
    return f"""module {{
  func.func @gather_literal() attributes {{grid = [1, 1]}} {{
    %xa = arith.constant 0 : index
    %i1a = arith.constant 32 : index
    %i2a = arith.constant 64 : index
    %ya = arith.constant 192 : index
    %c0 = arith.constant 0 : index
{views}
    %g = ktdp.construct_indirect_access_tile intermediate_variables(%m, %k)
        %xv[ind(%i1v[%m, %k]), ind(%i2v[%m, %k])] {{
      variables_space_set = {cs},
      variables_space_order = affine_map<(d0, d1) -> (d0, d1)>
    }} : memref<4x4xf16>, memref<4x4xi32>, memref<4x4xi32> -> !ktdp.access_tile<4x4xindex>
{configs._tile("yt", "yv", ["%c0", "%c0"], [4, 4], [4, 4], "f16")}
    %v = ktdp.load %g : !ktdp.access_tile<4x4xindex> -> tensor<4x4xf16>
    ktdp.store %v, %yt : tensor<4x4xf16>, !ktdp.access_tile<4x4xindex>
    return
  }}
}}
"""


def test_seeded_sticks_indirect_gather_golden():
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    interp = KTIRInterpreter()
    interp.load(_gather_4x4_literal())
    orig = interp._prepare_execution

    def prepare_and_seed(grid):
        orig(grid)
        hbm = interp.memory.hbm
        hbm.write(0, np.arange(16, dtype=np.float16))
        hbm.write(1, np.tile(np.array([3, 2, 1, 0], np.int32), 4))
        hbm.write(2, np.tile(np.array([0, 1, 2, 3], np.int32), 4))
        hbm.write(3, np.zeros(16, np.float16))

    interp._prepare_execution = prepare_and_seed
    assert interp.execute_function("gather_literal") == {}
    y = interp.memory.hbm.read(3, 16, "f16").reshape(4, 4)
    np.testing.assert_array_equal(y, np.tile(np.array([12, 9, 6, 3], np.float16), (4, 1)))
    # the seeded inputs are untouched, reads past an allocation's end are zero,
    # and an address in no allocation raises
    np.testing.assert_array_equal(interp.memory.hbm.read(0, 20, "f16"),
                                  np.concatenate([np.arange(16), np.zeros(4)]).astype(np.float16))
    with pytest.raises(ValueError):
        interp.memory.hbm.read(100, 4, "f16")


def test_seeded_table_beside_pointer_arguments():
    """A kernel reading one tensor from a literal address (seeded at stick 8)
    and the others from pointer arguments (placed from 0x10000 on)."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    n, blk = 1024, 256
    src, fn, names = _cases.elementwise(["%r = arith.addf %a, %t : {T_f16}"], ["f16"], "f16", n=n)
    lit = "\n".join(["    %ta = arith.constant 512 : index",
                     configs._view("t_view", "ta", [n], [1], "f16"),
                     configs._tile("t_t", "t_view", ["%off"], [blk], [n], "f16"),
                     f"    %t = ktdp.load %t_t : !ktdp.access_tile<{blk}xindex> -> tensor<{blk}xf16>"])
    src = src.replace("    %r = arith.addf", lit + "\n    %r = arith.addf")
    rng = np.random.default_rng(6)
    a, t = (rng.standard_normal(n).astype(np.float16) for _ in range(2))
    interp = KTIRInterpreter()
    interp.load(src)
    orig = interp._prepare_execution

    def prepare_and_seed(grid):
        orig(grid)
        interp.memory.hbm.write(8, t)

    interp._prepare_execution = prepare_and_seed
    out = interp.execute_function(fn, a_ptr=a, r_ptr=np.zeros(n, np.float16))
    np.testing.assert_array_equal(out["r_ptr"], a + t)
    np.testing.assert_array_equal(out["a_ptr"], a)
    # pointer arguments sit where the reference's allocator puts them
    r_stick = interp.memory.hbm.next_ptr // 128 - (n * 2) // 128
    np.testing.assert_array_equal(interp.memory.hbm.read(r_stick, n, "f16"), a + t)


def test_arg_names_and_sizes_drive_the_inputs():
    """The reference callers' pattern: names from arg_names, the length from
    tensor_input_output_sizes, then execute_function by those names."""
    from ktir_cpu_amd.interpreter import KTIRInterpreter
    interp = KTIRInterpreter()
    interp.load(configs.vector_add(4096, 128, 32))
    x_ptr, y_ptr, output_ptr, block = interp.arg_names("add_kernel")
    sizes = interp.tensor_input_output_sizes("add_kernel")
    assert sizes[x_ptr] == {"shape": (4096,), "dtype": "f16"}
    (n,) = sizes[x_ptr]["shape"]
    rng = np.random.default_rng(42)
    x, y = rng.standard_normal(n).astype(np.float16), rng.standard_normal(n).astype(np.float16)
    out = interp.execute_function("add_kernel", **{x_ptr: x, y_ptr: y, output_ptr: np.zeros(n, np.float16),
                                                   block: 128})
    np.testing.assert_array_equal(out[output_ptr], x + y)
    # positional remap: keys that name no argument, as many as the arguments
    out2 = interp.execute_function("add_kernel", a=x, b=y, c=np.zeros(n, np.float16), d=128)
    np.testing.assert_array_equal(out2[output_ptr], x + y)
