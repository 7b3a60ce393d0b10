"""Write tests/golden/m2_decode_cli.json from the reference's sources, read
as text (nothing of the reference is imported or run):

* flags: every `--flag` the decoder's parse loop accepts
  (native/fideslib_stage0/src/stage1_mamba2_config.cpp, `arg == "--x"`);
* defaults: every Config member initializer
  (native/fideslib_stage0/src/stage1_mamba2_config.hpp);
* messages: every std::invalid_argument message of parse_args;
* runner_argv: the campaign argv the runner passes
  (src/fhemamba/models/mamba2.py:40-75 builds it with
  experiments/dgx_mamba2_common.sh build_dgx_mamba2_args under the
  defaults of init_dgx_mamba2_defaults overlaid with the campaign's
  experiments/manifests/dgx_spark_stabilized_generation.json defaults and
  INPUT_CHAIN=payload), with {layers} and {tokens} left as placeholders;
* acceptance: that campaign's acceptance criteria.

    python tests/golden/make_m2_decode_cli_fixture.py [/root/reference]
"""
import json
import os
import re
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "m2_decode_cli.json")


def read(rel):
    with open(os.path.join(REF, rel)) as f:
        return f.read()


def main():
    cpp = read("native/fideslib_stage0/src/stage1_mamba2_config.cpp")
    hpp = read("native/fideslib_stage0/src/stage1_mamba2_config.hpp")
    sh = read("experiments/dgx_mamba2_common.sh")
    manifest = json.loads(read("experiments/manifests/dgx_spark_stabilized_generation.json"))

    parse = cpp[cpp.index("auto parse_args("):]
    flags = sorted(set(re.findall(r'arg == "(--[a-z0-9-]+)"', parse)))
    messages = sorted(set(
        m.replace('\\"', '"') for m in re.findall(
            r'std::invalid_argument\(\s*"((?:[^"\\]|\\.)*)"\s*\)', parse)))

    body = hpp[hpp.index("struct Config {"):hpp.index("};", hpp.index("struct Config {"))]
    body = re.sub(r"//[^\n]*", "", body)
    defaults = {}
    for typ, name, val in re.findall(
            r"(std::string|int|double|bool)\s+([a-z0-9_]+)\s*=\s*([^;]+);", body):
        val = val.strip()
        if typ == "std::string":
            defaults[name] = json.loads(val)
        elif typ == "int":
            defaults[name] = int(val)
        elif typ == "double":
            defaults[name] = float(val)
        else:
            defaults[name] = val == "true"
    for typ, name in re.findall(r"(std::string|std::set<int>)\s+([a-z0-9_]+)\s*;", body):
        defaults[name] = "" if typ == "std::string" else []

    init = sh[sh.index("init_dgx_mamba2_defaults() {"):sh.index("build_dgx_mamba2_args() {")]
    env = dict(re.findall(r'^\s*([A-Z0-9_]+)="\$\{\1:-([^}]*)\}"', init, re.M))
    env.update(manifest["defaults"])
    env["INPUT_CHAIN"] = "payload"
    build = sh[sh.index("build_dgx_mamba2_args() {"):]
    build = build[:build.index(")\n}")]
    pairs = re.findall(r'(--[a-z0-9-]+)\s+("\$[A-Z0-9_]+"|"\$layers"|"\$tokens"|\S+)', build)
    argv = []
    for flag, val in pairs:
        if val == '"$layers"':
            val = "{layers}"
        elif val == '"$tokens"':
            val = "{tokens}"
        elif val.startswith('"$'):
            name = val[2:-1]
            if name not in env:
                raise SystemExit(f"no default for {name}")
            val = env[name]
        argv.append([flag, val])

    out = {"source": {"parser": "native/fideslib_stage0/src/stage1_mamba2_config.cpp",
                      "config": "native/fideslib_stage0/src/stage1_mamba2_config.hpp",
                      "argv": "experiments/dgx_mamba2_common.sh build_dgx_mamba2_args",
                      "campaign": "experiments/manifests/dgx_spark_stabilized_generation.json"},
           "flags": flags, "defaults": defaults, "messages": messages,
           "runner_argv": argv, "acceptance": manifest["acceptance"]}
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"{OUT}: {len(flags)} flags, {len(defaults)} defaults, {len(messages)} messages, "
          f"{len(argv)} argv pairs")


if __name__ == "__main__":
    main()
