"""The small-batch kernel's prologue waits with an explicit vmcnt for its
record copy (global-to-LDS) while its first weight loads stay in flight.  That
is correct only if the copy is issued before every counted load and the count
equals the vector loads issued after the copy: vector loads retire in order.
This test compiles csrc/w4_limb.hip for gfx950 and checks both facts in the
assembly of every instantiation (a compiler that reordered or merged those
loads would make the wait return before the copy landed)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc")
                                    else shutil.which("hipcc"))


def vmcnt(line):
    m = re.search(r"vmcnt\((\d+)\)", line)
    return int(m.group(1)) if m else None


@pytest.mark.skipif(not HIPCC, reason="hipcc is not installed")
def test_limb_prologue_wait_counts_the_loads_after_the_record_copy(tmp_path):
    from torchburn_amd import build
    out = tmp_path / "w4_limb.s"
    src = os.path.join(ROOT, "torchburn_amd", "csrc", "w4_limb.hip")
    flags = [f for f in build.HIPCC_FLAGS if f not in ("-fPIC",)]
    cmd = [HIPCC, *flags, *build.EXTRA_FLAGS.get("w4_limb.hip", []), "-I", ROOT,
           "--cuda-device-only", "-S", src, "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    asm = out.read_text()
    names = re.findall(r"^(_ZN\w*k_w4_limb\w*):", asm, re.M)
    assert names, "no k_w4_limb instantiation found"
    for name in names:
        body = asm[asm.index(name + ":"):asm.index(".Lfunc_end", asm.index(name + ":"))]
        ins = [l.strip() for l in body.splitlines()
               if l.strip() and not l.strip().startswith((";", "."))]
        bar = next(i for i, l in enumerate(ins) if l.startswith("s_barrier"))
        pro = ins[:bar]
        dma = [i for i, l in enumerate(pro) if l.startswith("global_load_lds")]
        assert dma, name
        loads = [i for i, l in enumerate(pro) if l.startswith("global_load") and "_lds" not in l]
        assert all(i > max(dma) for i in loads), f"{name}: a load precedes the record copy"
        wait = [i for i, l in enumerate(pro) if l.startswith("s_waitcnt") and vmcnt(l) is not None]
        assert wait and wait[-1] > max(dma), name
        after = [i for i in loads if i < wait[-1]]
        assert vmcnt(pro[wait[-1]]) == len(after), \
            f"{name}: wait {pro[wait[-1]]} for {len(after)} loads after the copy"
