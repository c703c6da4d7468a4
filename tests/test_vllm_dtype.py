"""kvq.vllm_dtype: registering kv_cache_dtype="int8_static" in an installed vLLM (the registration the
reference applies as patches/vllm-0.32.0-int8-static-kv.patch:1-42). vLLM is not installed here, so
each test writes a small vLLM-shaped package (the three tables, laid out as vLLM lays them out),
registers the dtype, imports the edited modules and checks what vLLM would see: the name in the
CacheDType Literal, torch.int8 as its cache dtype, a new KVQuantMode member past the existing ones and
the string -> mode mapping, with every earlier mapping unchanged."""
import importlib.util
import os
import typing

import pytest
import torch

from kvq import vllm_dtype as vd

CACHE_PY = '''from typing import Literal

CacheDType = Literal[
    "auto",
    "bfloat16",
    "fp8",
    "fp8_e4m3",
    "int8_per_token_head",
    "nvfp4",
    "nvfp4_4over6",  # NVFP4 with the 4-over-6 scale rule
]
'''

TORCH_UTILS_PY = '''import torch

STR_DTYPE_TO_TORCH_DTYPE = {
    "float32": torch.float32,
    "half": torch.half,
    "bfloat16": torch.bfloat16,
    "fp8": torch.uint8,
    "int8": torch.int8,
    "int8_per_token_head": torch.int8,
    "nvfp4": torch.uint8
}
'''

KV_IFACE_PY = '''import enum


class KVQuantMode(enum.IntEnum):
    NONE = 0
    FP8 = 1
    INT8_PER_TOKEN_HEAD = 5
    NVFP4 = 7
    NVFP4_4OVER6 = 11  # packed FP4 with group scales

    @property
    def is_fp4(self) -> bool:
        return self in (KVQuantMode.NVFP4, KVQuantMode.NVFP4_4OVER6)


def get_kv_quant_mode(
    kv_cache_dtype: str,
) -> KVQuantMode:
    if kv_cache_dtype == "auto":
        return KVQuantMode.NONE
    if kv_cache_dtype.startswith("fp8"):
        return KVQuantMode.FP8
    if kv_cache_dtype == "int8_per_token_head":
        return KVQuantMode.INT8_PER_TOKEN_HEAD
    if kv_cache_dtype == "nvfp4_4over6":
        return KVQuantMode.NVFP4_4OVER6
    if kv_cache_dtype.startswith("nvfp4"):
        return KVQuantMode.NVFP4
    raise ValueError(kv_cache_dtype)
'''


def make_tree(root, cache=CACHE_PY, torch_utils=TORCH_UTILS_PY, iface=KV_IFACE_PY):
    pkg = os.path.join(str(root), "vllm")
    for rel, text in ((vd.FILES["cache_dtype"], cache), (vd.FILES["torch_dtype"], torch_utils),
                      (vd.FILES["quant_mode"], iface)):
        path = os.path.join(pkg, rel)
        os.makedirs(os.path.dirname(path), exist_ok=True)
        with open(path, "w") as f:
            f.write(text)
    return pkg


def load(pkg, key, tag):
    spec = importlib.util.spec_from_file_location(f"_vllm_{key}_{tag}", os.path.join(pkg, vd.FILES[key]))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def snapshot(pkg):
    out = {}
    for rel in vd.FILES.values():
        with open(os.path.join(pkg, rel)) as f:
            out[rel] = f.read()
    return out


def test_registers_int8_static_where_vllm_looks(tmp_path):
    pkg = make_tree(tmp_path)
    before = {k: load(pkg, k, "before") for k in vd.FILES}
    assert vd.status(pkg) == {"cache_dtype": False, "torch_dtype": False, "quant_mode": False}
    written = vd.install(pkg)
    assert len(written) == 3 and vd.status(pkg) == {k: True for k in vd.FILES}

    cache = load(pkg, "cache_dtype", "after")
    names = typing.get_args(cache.CacheDType)
    assert names[:-1] == typing.get_args(before["cache_dtype"].CacheDType) and names[-1] == "int8_static"

    tu = load(pkg, "torch_dtype", "after")
    assert tu.STR_DTYPE_TO_TORCH_DTYPE["int8_static"] is torch.int8
    assert {k: v for k, v in tu.STR_DTYPE_TO_TORCH_DTYPE.items() if k != "int8_static"} == \
        before["torch_dtype"].STR_DTYPE_TO_TORCH_DTYPE

    kv = load(pkg, "quant_mode", "after")
    old_modes = {m.name: int(m) for m in before["quant_mode"].KVQuantMode}
    assert int(kv.KVQuantMode.INT8_STATIC) == max(old_modes.values()) + 1 == 12
    assert {m.name: int(m) for m in kv.KVQuantMode if m.name != "INT8_STATIC"} == old_modes
    assert kv.get_kv_quant_mode("int8_static") is kv.KVQuantMode.INT8_STATIC
    assert not kv.KVQuantMode.INT8_STATIC.is_fp4          # the class body after the members is intact
    for s in ("auto", "fp8", "fp8_e4m3", "int8_per_token_head", "nvfp4", "nvfp4_4over6"):
        assert kv.get_kv_quant_mode(s).name == before["quant_mode"].get_kv_quant_mode(s).name, s
    with pytest.raises(ValueError):
        kv.get_kv_quant_mode("int4_static")


def test_second_install_changes_nothing(tmp_path):
    pkg = make_tree(tmp_path)
    vd.install(pkg)
    once = snapshot(pkg)
    assert vd.install(pkg) == [] and snapshot(pkg) == once


def test_one_line_tables_and_no_trailing_comma(tmp_path):
    cache = 'from typing import Literal\nCacheDType = Literal["auto", "fp8"]\n'
    tu = 'import torch\nSTR_DTYPE_TO_TORCH_DTYPE: dict[str, torch.dtype] = {"half": torch.half, "fp8": torch.uint8}\n'
    pkg = make_tree(tmp_path, cache=cache, torch_utils=tu)
    vd.install(pkg)
    assert typing.get_args(load(pkg, "cache_dtype", "one").CacheDType) == ("auto", "fp8", "int8_static")
    assert load(pkg, "torch_dtype", "one").STR_DTYPE_TO_TORCH_DTYPE == {
        "half": torch.half, "fp8": torch.uint8, "int8_static": torch.int8}
    with open(os.path.join(pkg, vd.FILES["cache_dtype"])) as f:
        assert 'Literal["auto", "fp8", "int8_static"]' in f.read()
    pkg2 = make_tree(tmp_path / "trailing", cache='from typing import Literal\nCacheDType = Literal["auto",]\n')
    vd.install(pkg2)
    assert typing.get_args(load(pkg2, "cache_dtype", "trail").CacheDType) == ("auto", "int8_static")


def test_missing_table_writes_nothing(tmp_path):
    iface = KV_IFACE_PY.replace("class KVQuantMode", "class CacheQuantMode")
    pkg = make_tree(tmp_path, iface=iface)
    before = snapshot(pkg)
    with pytest.raises(vd.PatchError, match="KVQuantMode"):
        vd.install(pkg)
    assert snapshot(pkg) == before                       # the two editable files were left alone too
    with pytest.raises(vd.PatchError, match="missing"):
        vd.install(str(tmp_path))                        # not a vllm package directory


def test_cli_check_and_install(tmp_path, capsys):
    pkg = make_tree(tmp_path)
    assert vd.main(["--vllm-root", pkg, "--check"]) == 1
    assert "NOT registered" in capsys.readouterr().out
    assert vd.main(["--vllm-root", pkg]) == 0
    assert vd.main(["--vllm-root", pkg, "--check"]) == 0
    assert vd.main(["--vllm-root", str(tmp_path)]) == 2


def test_missing_tables_names_what_the_plugin_warns_about(tmp_path):
    pkg = make_tree(tmp_path)
    assert vd.missing_tables(pkg) == list(vd.FILES.values())
    vd.install(pkg)
    assert vd.missing_tables(pkg) == []
    assert vd.missing_tables(str(tmp_path)) is None     # not a vLLM source tree: the plugin stays quiet


@pytest.mark.parametrize("stage", ["write", "replace"])
def test_failed_install_leaves_vllm_as_it_was(tmp_path, monkeypatch, stage):
    """An I/O failure part-way through install() -- writing the second edited file, or moving the second
    into place after the first was replaced -- leaves all three tables as they were and no temporary
    files behind, then re-raises."""
    pkg = make_tree(tmp_path)
    before = snapshot(pkg)
    if stage == "write":
        real_open = open
        calls = []

        def failing_open(path, mode="r", *a, **k):
            if str(path).endswith(".kvq-tmp") and "w" in mode:
                calls.append(path)
                if len(calls) == 2:
                    raise OSError(28, "No space left on device")
            return real_open(path, mode, *a, **k)
        monkeypatch.setattr("builtins.open", failing_open)
    else:
        real_replace = vd._replace
        done = []

        def failing_replace(src, dst):
            if done:
                raise PermissionError(13, "Permission denied", dst)
            real_replace(src, dst)
            done.append(dst)
        monkeypatch.setattr(vd, "_replace", failing_replace)
    with pytest.raises(OSError):
        vd.install(pkg)
    monkeypatch.undo()
    assert snapshot(pkg) == before
    leftovers = [f for _, _, fs in os.walk(pkg) for f in fs if f.endswith(".kvq-tmp")]
    assert leftovers == []
    assert vd.missing_tables(pkg) == list(vd.FILES.values())


def test_missing_tables_stays_quiet_on_unreadable_sources(tmp_path):
    """missing_tables() is the plugin's warning: an unreadable or undecodable vLLM source is reported as
    'not a table tree' (None), never raised into vLLM's plugin loading."""
    pkg = make_tree(tmp_path)
    with open(os.path.join(pkg, vd.FILES["torch_dtype"]), "wb") as f:
        f.write(b"\xff\xfe\x00 not utf-8 \x80\x81")
    assert vd.missing_tables(pkg) is None
    os.remove(os.path.join(pkg, vd.FILES["torch_dtype"]))
    os.mkdir(os.path.join(pkg, vd.FILES["torch_dtype"]))    # a directory where the file should be
    assert vd.missing_tables(pkg) is None
