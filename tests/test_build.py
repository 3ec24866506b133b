"""The build recipe refuses kernels that fall back to scratch memory (CPU only)."""
import importlib.util
import os

_spec = importlib.util.spec_from_file_location(
    "q3a_build", os.path.join(os.path.dirname(__file__), "..", "qwen3-tts-engine_amd", "build.py"))
build = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(build)

REMARKS = """\
a.hip:10:1: remark: Function Name: kernel_a
a.hip:10:1: remark:     SGPRs: 40
a.hip:10:1: remark:     VGPRs: 103
a.hip:10:1: remark:     ScratchSize [bytes/lane]: 304
   10 | __global__ void kernel_a() {
      | ^
a.hip:20:1: remark: Function Name: kernel_b
a.hip:20:1: remark:     ScratchSize [bytes/lane]: 0
"""


def test_scratch_users_names_only_the_spilling_kernel():
    assert build.scratch_users(REMARKS) == ["kernel_a (304 B/lane)"]
    assert build.scratch_users("") == []
