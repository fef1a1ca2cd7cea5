"""The kernel hashes (alphazero-go_amd/build.py: kernel_hash, conv_hash) name
the sources and flags of a build, not where the checkout lies: two copies of
the tree at different paths hash alike, and a changed kernel source does not.
bench.py keys the committed counter summaries by the convolution's hash, so a
library built from the same files anywhere finds them."""
import importlib.util
import os
import shutil

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "alphazero-go_amd")


def _copy_tree(dest):
    shutil.copytree(os.path.join(PKG, "csrc"), os.path.join(dest, "alphazero-go_amd", "csrc"))
    shutil.copy(os.path.join(PKG, "build.py"), os.path.join(dest, "alphazero-go_amd", "build.py"))
    shutil.copytree(os.path.join(ROOT, "include"), os.path.join(dest, "include"))
    return os.path.join(dest, "alphazero-go_amd", "build.py")


def _load(path, name):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_hash_independent_of_checkout_path(tmp_path):
    here = _load(os.path.join(PKG, "build.py"), "build_here")
    a = _load(_copy_tree(str(tmp_path / "a")), "build_a")
    b = _load(_copy_tree(str(tmp_path / "deeper" / "checkout" / "b")), "build_b")
    assert a.ROOT != b.ROOT != here.ROOT
    assert a.kernel_hash() == b.kernel_hash() == here.kernel_hash()
    assert a.conv_hash() == b.conv_hash() == here.conv_hash()


def test_hash_follows_the_sources(tmp_path):
    a = _load(_copy_tree(str(tmp_path / "a")), "build_a2")
    before_kernel, before_conv = a.kernel_hash(), a.conv_hash()
    with open(os.path.join(a.CSRC, "azh_conv.hpp"), "a") as f:
        f.write("\n// a changed convolution source\n")
    assert a.conv_hash() != before_conv and a.kernel_hash() != before_kernel
    with open(os.path.join(a.ROOT, "include", "azgo_hip.h"), "a") as f:
        f.write("\n/* a changed header */\n")
    after_conv = a.conv_hash()
    assert a.kernel_hash() != before_kernel
    with open(os.path.join(a.CSRC, "azh_kernels.hip"), "a") as f:
        f.write("\n// a changed head kernel\n")
    assert a.conv_hash() == after_conv, "the convolution's hash covers its own sources only"
