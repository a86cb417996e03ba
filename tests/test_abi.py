"""The device library loads and exports every symbol include/q3t_dev.h
declares; without a HIP device it refuses to create a context (no CPU
fallback).  No compute call is made here."""
import ctypes
import os
import re

import pytest

from qwen3_tts_amd import config
from qwen3_tts_amd.device import EXPORTS, LIB_PATH, Device, DeviceError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q3t_dev.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q3t_dev_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    assert declared_functions() == sorted(EXPORTS)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "build() first"
    lib = ctypes.CDLL(LIB_PATH)
    missing = [f for f in declared_functions() if not hasattr(lib, f)]
    assert not missing, missing


def test_no_device_no_fallback():
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from qwen3_tts_amd import config\n"
            "from qwen3_tts_amd.device import Device, DeviceError\n"
            "try:\n    Device(config.tiny())\nexcept DeviceError as e:\n    print('refused:', e)\n"
            "else:\n    print('created')\n") % os.path.join(ROOT, "qwen3-tts.cpp_amd")
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert "refused:" in out.stdout, out.stdout + out.stderr


def test_config_struct_matches_header_field_count():
    text = open(HEADER).read()
    body = text[text.index("typedef struct q3t_config {"):text.index("} q3t_config;")]
    decls = [l for l in body.splitlines()[1:] if ";" in l]
    n = sum(len(l.split(";")[0].split(",")) for l in decls)
    assert n == len(config.CConfig._fields_)
    assert ctypes.sizeof(config.CConfig) == 4 * n


VOC_HEADER = os.path.join(ROOT, "include", "q3t_voc.h")


def test_vocoder_header_declares_the_bound_functions():
    from qwen3_tts_amd.vocoder import VOC_EXPORTS
    text = re.sub(r"/\*.*?\*/", "", open(VOC_HEADER).read(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(q3t_voc_[a-z_0-9]+)\s*\(", text)))
    assert declared == sorted(VOC_EXPORTS)
    lib = ctypes.CDLL(LIB_PATH)
    missing = [f for f in declared if not hasattr(lib, f)]
    assert not missing, missing


def test_vocoder_config_struct_matches_header():
    from qwen3_tts_amd import vocoder
    text = open(VOC_HEADER).read()
    body = text[text.index("typedef struct q3t_voc_config {"):text.index("} q3t_voc_config;")]
    names = re.findall(r"\b([a-z_]+)(?:\[\d\])?;", body)
    assert names == [n for n, _ in vocoder.CVocConfig._fields_]


def test_vocoder_refuses_without_device():
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from qwen3_tts_amd import vocoder as V\n"
            "try:\n    V.VocDevice(V.tiny(), V.VocWeights(V.tiny()))\nexcept V.VocError as e:\n    print('refused:', e)\n"
            "else:\n    print('created')\n") % os.path.join(ROOT, "qwen3-tts.cpp_amd")
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert "refused:" in out.stdout, out.stdout + out.stderr
