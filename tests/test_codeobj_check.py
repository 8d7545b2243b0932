"""Build-time guard for the untracked LDS DMA of the packed-weight MoE kernels.

The pipelines in csrc/w4pk.h issue ``buffer_load ... lds`` as inline assembly
that the compiler's wait pass does not see, which is only correct while those
kernels use no scratch (a spill reload's wait would reorder the DMA) and while
the assembly keeps its hazard padding. These CPU tests compile small kernels
with hipcc (no GPU) and check that ``intent_amd.build.build`` rejects the bad
ones and passes the library's own objects.
"""
import shutil
from pathlib import Path

import pytest

from intent_amd import build as B
from intent_amd import codeobj_check as C

pytestmark = pytest.mark.skipif(shutil.which(B.hipcc()) is None and not Path(B.hipcc()).exists(),
                                reason="hipcc not available")

_CSRC = str(B.CSRC)

# A kernel named like a registered untracked-DMA kernel, using the library's
# own assembly DMA, with a VGPR budget small enough to force spills.
_SPILLING = r'''
#include "mfma_pipe.h"
extern "C" __global__ __attribute__((amdgpu_num_vgpr(24))) __launch_bounds__(256)
void moe_gate_up_pk_kernel_spill_case(const float* __restrict__ p, int n, float* __restrict__ out) {
  __shared__ float buf[4096];
  mp::Rsrc rs = make_rsrc(p);
  float acc[48];
#pragma unroll
  for (int i = 0; i < 48; ++i) acc[i] = p[threadIdx.x + 256 * i];
  for (int it = 0; it < n; ++it) {
    mp::lds_dma<16, true>(rs, (mp::lds_t*)(buf + 256 * (it & 3)), threadIdx.x * 16, it * 4096);
#pragma unroll
    for (int i = 0; i < 48; ++i) acc[i] = acc[i] * acc[(i + 7) % 48] + buf[(threadIdx.x + i) & 4095];
    __syncthreads();
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 48; ++i) s += acc[i];
  out[threadIdx.x] = s;
}
'''

# The same DMA with no register pressure: accepted.
_CLEAN = r'''
#include "mfma_pipe.h"
extern "C" __global__ __launch_bounds__(256)
void moe_gate_up_pk_kernel_clean_case(const float* __restrict__ p, int n, float* __restrict__ out) {
  __shared__ float buf[4096];
  mp::Rsrc rs = make_rsrc(p);
  for (int it = 0; it < n; ++it) {
    mp::lds_dma<16, true>(rs, (mp::lds_t*)(buf + 1024 * (it & 3)), threadIdx.x * 16, it * 4096);
    mp::wait_vm<0>();
    __syncthreads();
  }
  out[threadIdx.x] = buf[threadIdx.x];
}
'''

# Assembly DMA written without the M0 wait state: rejected.
_NO_NOP = r'''
#include "mfma_pipe.h"
extern "C" __global__ __launch_bounds__(256)
void m0_hazard_case(const float* __restrict__ p, int n, float* __restrict__ out) {
  __shared__ float buf[1024];
  mp::Rsrc rs = make_rsrc(p);
  for (int it = 0; it < n; ++it) {
    const uint32_t m = (uint32_t)(uintptr_t)(mp::lds_t*)(buf + 64 * (it & 3));
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                 : : "s"(m), "v"(threadIdx.x * 4), "s"(rs), "s"(it * 256) : "memory");
  }
  mp::wait_vm<0>();
  __syncthreads();
  out[threadIdx.x] = buf[threadIdx.x];
}
'''


def _build(tmp_path, name, text):
    src = tmp_path / f"{name}.hip"
    src.write_text(text)
    return B.build(sources=[src], extra_flags=[f"-I{_CSRC}"], library=tmp_path / f"lib{name}.so",
                   objdir=tmp_path / name)


def test_spilling_untracked_dma_kernel_is_rejected(tmp_path):
    with pytest.raises(C.CodeObjectError, match="spill|scratch|private segment"):
        _build(tmp_path, "spill", _SPILLING)


def test_clean_untracked_dma_kernel_builds(tmp_path):
    lib = _build(tmp_path, "clean", _CLEAN)
    assert lib.exists()


def test_missing_m0_wait_state_is_rejected(tmp_path):
    with pytest.raises(C.CodeObjectError, match="M0"):
        _build(tmp_path, "nonop", _NO_NOP)


def test_library_packed_moe_kernels_pass_the_check(tmp_path):
    """The library's own moe.hip: its packed-weight kernels are found, carry
    LDS DMA and pass (no scratch, padded hazards)."""
    obj = B._compile(B.CSRC / "moe.hip", tmp_path)
    reports = C.check_binary(obj, tmp_path / "co")
    for k in C.UNTRACKED_DMA_KERNELS:
        found = [r for r in reports if k in r.name]
        assert found, k
        assert all(r.dma > 0 and r.spills == 0 and r.private_segment == 0 and r.scratch_ops == 0 for r in found)


def test_valu_sgpr_write_parser():
    assert C._valu_sgpr_writes("v_readfirstlane_b32 s7, v3") == {"s7"}
    assert C._valu_sgpr_writes("v_cmp_gt_i32_e32 vcc, s6, v11") == {"vcc"}
    assert C._valu_sgpr_writes("v_mad_u64_u32 v[20:21], s[2:3], v11, s10, v[20:21]") == {"s2", "s3"}
    assert C._valu_sgpr_writes("v_or_b32_e32 v11, s7, v9") == set()
    assert C._dma_sgpr_reads("buffer_load_dwordx4 v8, s[24:27], s2 offen lds") == {"s24", "s25", "s26", "s27", "s2"}
