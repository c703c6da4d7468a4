"""Register kv_cache_dtype="int8_static" in an installed vLLM (ROCm and CUDA builds alike: the change
touches vLLM's Python sources only).

vLLM checks `kv_cache_dtype` against three tables of its own before any attention backend is asked,
so the static INT8 backend needs its name in each. The reference ships the same registration as a
source diff for vLLM 0.32.0 applied when its image is built (patches/vllm-0.32.0-int8-static-kv.patch:1-42):

* vllm/config/cache.py          -- the `CacheDType` Literal the cache config is validated against;
* vllm/utils/torch_utils.py     -- `STR_DTYPE_TO_TORCH_DTYPE`, which types the cache: int8_static -> torch.int8;
* vllm/v1/kv_cache_interface.py -- a `KVQuantMode` member for it, and its case in the function that maps
  a cache dtype string to its mode (placed first, ahead of prefix tests such as "nvfp4").

Instead of a diff pinned to one release's lines, each edit finds its table by name and appends the
entry, so it applies to any vLLM release that has these tables. Nothing is written unless all three
files can be edited (a missing table is an error naming it); applying twice changes nothing.

    python -m kvq.vllm_dtype                  # edit the vLLM that `import vllm` would load
    python -m kvq.vllm_dtype --check          # exit status 1 while it is not registered
    python -m kvq.vllm_dtype --vllm-root DIR  # edit the vLLM package in DIR
"""
import argparse
import importlib.util
import os
import re
import sys

NAME = "int8_static"
MODE = "INT8_STATIC"
FILES = {
    "cache_dtype": os.path.join("config", "cache.py"),
    "torch_dtype": os.path.join("utils", "torch_utils.py"),
    "quant_mode": os.path.join("v1", "kv_cache_interface.py"),
}


class PatchError(RuntimeError):
    pass


def find_vllm():
    """Directory of the vllm package `import vllm` would load (located without importing it)."""
    spec = importlib.util.find_spec("vllm")
    if spec is None or not spec.submodule_search_locations:
        raise PatchError("no importable vllm package in this environment; pass --vllm-root")
    return list(spec.submodule_search_locations)[0]


def _closing(text, i):
    """Index of the bracket closing the one at text[i], skipping string literals and comments."""
    pairs = {"[": "]", "{": "}", "(": ")"}
    stack = [pairs[text[i]]]
    j = i + 1
    while j < len(text):
        c = text[j]
        if c in "\"'":
            end = text.find(c, j + 1)
            if end < 0:
                break
            j = end
        elif c == "#":
            j = text.find("\n", j)
            if j < 0:
                break
        elif c in pairs:
            stack.append(pairs[c])
        elif c in ")]}":
            if c != stack.pop():
                break
            if not stack:
                return j
        j += 1
    raise PatchError("unbalanced brackets")


def _append_entry(text, header, entry, present, where):
    """Append `entry` inside the bracket that `header` (a regex ending at the opening bracket) opens,
    unless `present` already matches inside it. Multi-line bodies get a line of their own at the
    entries' indentation; one-line bodies get ", entry"."""
    m = re.search(header, text, re.M)
    if not m:
        raise PatchError(f"{where}: no match for {header!r}")
    open_i = m.end() - 1
    close_i = _closing(text, open_i)
    body = text[open_i + 1:close_i]
    if re.search(present, body):
        return text
    if "\n" not in body:
        sep = "" if not body.strip() else " " if body.rstrip().endswith(",") else ", "
        return text[:close_i].rstrip() + sep + entry + text[close_i:]
    lines = body.split("\n")
    code_lines = [i for i, ln in enumerate(lines) if ln.strip() and not ln.strip().startswith("#")]
    if not code_lines:
        raise PatchError(f"{where}: empty table")
    indent = re.match(r"[ \t]*", lines[code_lines[0]]).group(0)
    # the last entry must end in a comma (before any comment on its line) once another follows it
    li = code_lines[-1]
    code = re.sub(r"[ \t]*#.*$", "", lines[li]).rstrip()
    if not code.endswith(","):
        lines[li] = code + "," + lines[li][len(code):]
    # the new entry goes after the last non-blank line of the body (entries and trailing comments)
    tail = max(i for i, ln in enumerate(lines) if ln.strip())
    lines.insert(tail + 1, indent + entry + ",")
    return text[:open_i + 1] + "\n".join(lines) + text[close_i:]


def _edit_cache_dtype(text, where):
    return _append_entry(text, r"^CacheDType\s*=\s*Literal\[", f'"{NAME}"', rf'["\']{NAME}["\']', where)


def _edit_torch_dtype(text, where):
    return _append_entry(text, r"^STR_DTYPE_TO_TORCH_DTYPE\b[^=\n]*=\s*\{", f'"{NAME}": torch.int8',
                         rf'["\']{NAME}["\']\s*:', where)


def _block_end(text, start):
    """End of the top-level block (class / def) whose header line starts at `start`."""
    m = re.compile(r"^[A-Za-z_@]", re.M).search(text, text.index("\n", start) + 1)
    return m.start() if m else len(text)


def _edit_quant_mode(text, where):
    cm = re.search(r"^class KVQuantMode\b[^\n]*:[ \t]*\n", text, re.M)
    if not cm:
        raise PatchError(f"{where}: no class KVQuantMode")
    cend = _block_end(text, cm.start())
    members = list(re.finditer(r"^([ \t]+)([A-Z][A-Z0-9_]*)[ \t]*=[ \t]*(-?\d+)\b[^\n]*\n", text[:cend], re.M))
    members = [mm for mm in members if mm.start() >= cm.end()]
    if not members:
        raise PatchError(f"{where}: KVQuantMode has no integer members")
    if not any(mm.group(2) == MODE for mm in members):
        value = max(int(mm.group(3)) for mm in members) + 1
        last = members[-1]
        line = f"{last.group(1)}{MODE} = {value}  # int8 codes; calibrated static scales held by the attention backend\n"
        text = text[:last.end()] + line + text[last.end():]
    # the function mapping a cache dtype string to its KVQuantMode: the top-level def whose body
    # returns KVQuantMode members; its first parameter is the dtype string
    for fm in re.finditer(r"^def \w+\(\s*(\w+)[^\n]*\n", text, re.M):
        fend = _block_end(text, fm.start())
        body = text[fm.end():fend]
        if "return KVQuantMode." not in body:
            continue
        var = fm.group(1)
        if re.search(rf'\b{var}\s*==\s*["\']{NAME}["\']', body):
            return text
        im = re.search(rf"^([ \t]+)if\b[^\n]*\b{var}\b", body, re.M)
        if not im:
            raise PatchError(f"{where}: the dtype -> KVQuantMode function tests no `{var}`")
        ind = im.group(1)
        case = f'{ind}if {var} == "{NAME}":\n{ind}    return KVQuantMode.{MODE}\n'
        at = fm.end() + im.start()
        return text[:at] + case + text[at:]
    raise PatchError(f"{where}: no function returning KVQuantMode members")


EDITS = {"cache_dtype": _edit_cache_dtype, "torch_dtype": _edit_torch_dtype, "quant_mode": _edit_quant_mode}


def _plan(root):
    """{key: (path, old text, new text)} for the three files, or PatchError before anything is written."""
    out = {}
    for key, rel in FILES.items():
        path = os.path.join(root, rel)
        if not os.path.isfile(path):
            raise PatchError(f"{path}: missing (is {root} a vLLM package directory?)")
        with open(path, encoding="utf-8") as f:
            old = f.read()
        new = EDITS[key](old, path)
        try:
            compile(new, path, "exec")
        except SyntaxError as e:  # never leave vLLM unimportable
            raise PatchError(f"{path}: the edited file would not compile ({e})") from e
        out[key] = (path, old, new)
    return out


def status(root=None):
    """{table: True if int8_static is already registered there} for the vLLM package in `root`."""
    root = root or find_vllm()
    return {key: old == new for key, (_, old, new) in _plan(root).items()}


def install(root=None):
    """Register int8_static in the vLLM package in `root` (default: the importable one). Returns the
    paths written (empty when it was already registered). All or nothing: every edited file is written
    to a temporary file beside it first; only then are they moved into place, and if any step fails the
    temporary files are removed and the files already replaced get their original text back, so vLLM is
    never left with some of its tables registered."""
    root = root or find_vllm()
    todo = [(path, old, new) for path, old, new in _plan(root).values() if new != old]
    staged, replaced = [], []
    try:
        for path, old, new in todo:
            tmp = path + ".kvq-tmp"
            staged.append(tmp)
            with open(tmp, "w", encoding="utf-8") as f:
                f.write(new)
        for (path, old, new), tmp in zip(todo, staged):
            _replace(tmp, path)
            replaced.append((path, old))
    except BaseException:
        for tmp in staged:
            if os.path.exists(tmp):
                os.remove(tmp)
        for path, old in replaced:
            with open(path, "w", encoding="utf-8") as f:
                f.write(old)
        raise
    return [path for path, _, _ in todo]


def _replace(src, dst):
    os.replace(src, dst)


def missing_tables(root=None):
    """Paths (relative to the vllm package) of the tables that still lack int8_static, or None when
    `root` (default: the importable vllm) is not a source tree with these tables, or its files cannot be
    read or parsed (the plugin only warns: nothing here may stop vLLM from loading it)."""
    try:
        return [FILES[key] for key, ok in status(root).items() if not ok]
    except (PatchError, OSError, ValueError):   # (UnicodeDecodeError is a ValueError) -- a warning's worth
        return None


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m kvq.vllm_dtype", description=__doc__.split("\n\n")[0])
    ap.add_argument("--vllm-root", help="vllm package directory (default: the one `import vllm` loads)")
    ap.add_argument("--check", action="store_true", help="only report; exit status 1 if not registered")
    args = ap.parse_args(argv)
    try:
        root = args.vllm_root or find_vllm()
        st = status(root)
        if args.check:
            for key, ok in st.items():
                print(f"{FILES[key]}: {'registered' if ok else 'NOT registered'}")
            return 0 if all(st.values()) else 1
        written = install(root)
    except PatchError as e:
        print(f"error: {e}", file=sys.stderr)
        return 2
    for p in written:
        print(f"registered {NAME} in {p}")
    if not written:
        print(f"{NAME} already registered in {root}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
