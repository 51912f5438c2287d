"""The C++ drop-in API (vk_symbiote/*.h + libvsl_engine.so) as a reference application uses it:
programs under tests/cpp are compiled with g++ against the headers and linked with the engine
library.  The GGUFLoader check runs here (host code only); the engine program is compiled here and
run on the GPU by tests/test_engine_gpu.py."""
import os
import subprocess

import pytest

import vsl_testlib

ROOT = vsl_testlib.ROOT
CPP = os.path.join(ROOT, "tests", "cpp")


def compile_cpp(vsl, src, out):
    """g++ -std=c++17 <src> against vk_symbiote/*.h and include/, linked with libvsl_engine.so."""
    lib_dir = os.path.dirname(vsl.ENGINE_LIB)
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-Wno-unused-parameter",
           "-I", os.path.join(vsl_testlib.PKG_DIR, "csrc", "host", "vk_symbiote"), "-I", os.path.join(ROOT, "include"),
           os.path.join(CPP, src), "-o", str(out), f"-L{lib_dir}", "-lvsl_engine", f"-Wl,-rpath,{lib_dir}",
           "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return str(out)


def test_gguf_loader_cpp_api(vsl, tmp_path):
    """Every public GGUFLoader method of the reference header (GGUFLoader.h:265-333), including
    stream_tensors_parallel, get_vocabulary / get_tokenizer_config, the tensor cache methods and
    add_shard / is_sharded, on files written by GGUFWriter; and Expected<T>'s interface."""
    exe = compile_cpp(vsl, "gguf_api_check.cpp", tmp_path / "gguf_api_check")
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    for part in ("vocabulary ok", "metadata arrays ok", "shards ok", "stream ok", "cache ok", "expected ok"):
        assert part in r.stdout
    assert "checks passed" in r.stdout


def test_integration_program_compiles(vsl, tmp_path):
    """The C++ drop-in program (ConfigManager + VulkanSymbioteEngine(path) + generate + run_benchmark)
    compiles and links against the headers and libvsl_engine.so."""
    exe = compile_cpp(vsl, "integration_app.cpp", tmp_path / "integration_app")
    assert os.path.exists(exe)
