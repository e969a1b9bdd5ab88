"""The build refuses scratch memory in kernels that wait for LDS DMA with exact
vmcnt counts (marlin-mlx_amd/build.py): the remark parser must find every
function with a nonzero ScratchSize and nothing else."""
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build_module():
    spec = importlib.util.spec_from_file_location("mq4_build_guard", os.path.join(ROOT, "marlin-mlx_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


REMARKS = """\
k.hip:10:1: remark: Function Name: kern_a [-Rpass-analysis=kernel-resource-usage]
k.hip:10:1: remark:     VGPRs: 202 [-Rpass-analysis=kernel-resource-usage]
k.hip:10:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
k.hip:20:1: remark: Function Name: kern_b [-Rpass-analysis=kernel-resource-usage]
k.hip:20:1: remark:     VGPRs: 168 [-Rpass-analysis=kernel-resource-usage]
k.hip:20:1: remark:     ScratchSize [bytes/lane]: 132 [-Rpass-analysis=kernel-resource-usage]
k.hip:30:1: remark: Function Name: kern_c [-Rpass-analysis=kernel-resource-usage]
k.hip:30:1: remark:     ScratchSize [bytes/lane]: 4 [-Rpass-analysis=kernel-resource-usage]
"""


def test_scratch_users_parser():
    b = _build_module()
    assert b._scratch_users(REMARKS) == [("kern_b", 132), ("kern_c", 4)]
    assert b._scratch_users(REMARKS.replace(": 132 ", ": 0 ").replace(": 4 ", ": 0 ")) == []
    assert b._scratch_users("") == []


def test_guarded_sources():
    b = _build_module()
    # the two sources whose kernels wait for LDS DMA by exact vmcnt
    assert {"mq4_gemm.hip", "mq4_decode.hip"} <= b.NO_SCRATCH
