"""Generate g1_model_tables.h: the Unitree G1 model constants as constexpr C++ tables.

The numbers are physical data of the robot, produced by MuJoCo 3.9.0's model compiler from
models/g1.xml + models/scene.xml (BSD-3, Unitree / MuJoCo Menagerie). MuJoCo is not installed
here, so the only source for the compiled quantities (body_iquat, the diagonal body_inertia, the
damping-ratio-derived kd, body_invweight0) is the reference's own generated header
(reference: src/g1_model.h:5-474, written by scripts/export_model.py:44-184).  This script reads
that header as text, keeps every literal exactly as printed, and emits:

  * ModelT<float>  -- the literals with an `f` suffix (the values the fp32 device code uses),
  * ModelT<double> -- the same decimal literals as doubles (fp64 oracle instantiation),
  * integer topology tables (parent, dof/qpos addresses, actuator maps),
  * derived topology used by the lane-cooperative kernels (depth, children lists).

Run only where the reference tree is mounted; the output is committed, so nothing at build or
run time reads the reference.

    python g1.cu_amd/csrc/gen_model_tables.py [/root/reference/src/g1_model.h]
"""
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "g1_model_tables.h")
SRC_DEFAULT = "/root/reference/src/g1_model.h"

ARR_RE = re.compile(r"__device__\s+__constant__\s+(float|int)\s+(\w+)\[(\d+)\]\s*=\s*\{([^}]*)\};", re.S)
DEF_RE = re.compile(r"#define\s+(\w+)\s+(\S+)")

# reference table name -> our table name
FLOAT_TABLES = {
    "G1_GRAVITY": "gravity",
    "body_pos": "body_pos",
    "body_quat": "body_quat",
    "body_ipos": "body_ipos",
    "body_iquat": "body_iquat",
    "body_mass": "body_mass",
    "body_inertia": "body_inertia",
    "jnt_axis": "jnt_axis",
    "jnt_pos": "jnt_pos",
    "dof_armature": "dof_armature",
    "qpos0": "qpos0",
    "g1_qpos_stand": "qpos_stand",
    "g1_foot_lpos": "foot_lpos",
    "G1_FOOT_SOLREF": "foot_solref",
    "G1_FOOT_SOLIMP": "foot_solimp",
    "g1_foot_body_invweight0": "foot_invweight0",
    "g1_act_kp": "act_kp",
    "g1_act_kd": "act_kd",
    "g1_act_ctrl_lo": "act_ctrl_lo",
    "g1_act_ctrl_hi": "act_ctrl_hi",
    "g1_act_frc_lo": "act_frc_lo",
    "g1_act_frc_hi": "act_frc_hi",
}
INT_TABLES = {
    "body_parentid": "body_parent",
    "body_jntnum": "body_jntnum",
    "body_jntadr": "body_jntadr",
    "body_dofadr": "body_dofadr",
    "body_dofnum": "body_dofnum",
    "jnt_type": "jnt_type",
    "jnt_bodyid": "jnt_bodyid",
    "jnt_qposadr": "jnt_qposadr",
    "jnt_dofadr": "jnt_dofadr",
    "g1_foot_body": "foot_body",
    "g1_act_dof": "act_dof",
    "g1_act_qadr": "act_qadr",
}
FLOAT_DEFINES = {"G1_DT": "dt", "G1_FOOT_RADIUS": "foot_radius", "G1_FOOT_MU": "foot_mu",
                 "G1_FOOT_IMPRATIO": "foot_impratio"}
INT_DEFINES = {"G1_NBODY": "kNBody", "G1_NQ": "kNQ", "G1_NV": "kNV", "G1_NJNT": "kNJnt",
               "G1_NFOOT_SPHERE": "kNFoot", "G1_NU": "kNU", "G1_FOOT_CONDIM": "kFootCondim"}


def parse(path):
    text = open(path).read()
    arrays = {}
    for typ, name, n, body in ARR_RE.findall(text):
        vals = [v.strip() for v in body.replace("\n", " ").split(",") if v.strip()]
        assert len(vals) == int(n), (name, len(vals), n)
        arrays[name] = (typ, vals)
    defines = {k: v for k, v in DEF_RE.findall(text)}
    return arrays, defines


def flit(s, dbl):
    """Decimal literal as printed in the source, as a float (`f`) or double literal."""
    s = s.strip()
    if s.endswith("f"):
        s = s[:-1]
    if not any(c in s for c in ".eE"):
        s += ".0"
    return s if dbl else s + "f"


def emit_float_table(name, vals, dbl, ncol):
    typ = "double" if dbl else "float"
    lits = [flit(v, dbl) for v in vals]
    rows = [", ".join(lits[i:i + ncol]) for i in range(0, len(lits), ncol)]
    body = ",\n      ".join(rows)
    return f"  static constexpr {typ} {name}[{len(vals)}] = {{\n      {body}}};\n"


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else SRC_DEFAULT
    arrays, defines = parse(src)
    ints = {}
    for ref, ours in INT_TABLES.items():
        typ, vals = arrays[ref]
        assert typ == "int"
        ints[ours] = [int(v) for v in vals]
    idef = {ours: int(defines[ref]) for ref, ours in INT_DEFINES.items()}

    nb = idef["kNBody"]
    parent = ints["body_parent"]
    # Structural facts the kernels rely on; fail generation if the model ever changes shape.
    assert all(parent[b] < b for b in range(1, nb)), "parents must precede children"
    assert ints["body_jntnum"][1:] == [1] * (nb - 1), "exactly one joint per moving body"
    assert ints["jnt_type"][0] == 0 and all(t == 3 for t in ints["jnt_type"][1:]), "free + hinges"
    assert ints["body_dofnum"][1] == 6 and all(n == 1 for n in ints["body_dofnum"][2:])
    assert all(float(v.rstrip("f")) == 0.0 for v in arrays["jnt_pos"][1]), "hinge anchors at body origin"
    assert ints["body_dofadr"][2:] == [b + 4 for b in range(2, nb)]
    assert ints["jnt_qposadr"][1:] == [b + 6 for b in range(1, nb - 1)]
    assert ints["act_dof"] == [6 + i for i in range(idef["kNU"])]
    assert ints["act_qadr"] == [7 + i for i in range(idef["kNU"])]

    depth = [0] * nb
    for b in range(1, nb):
        depth[b] = depth[parent[b]] + 1
    children = [[c for c in range(nb - 1, 0, -1) if parent[c] == b] for b in range(nb)]
    maxchild = max(len(c) for c in children[1:])
    assert maxchild <= 3
    kids = [(c + [-1] * 3)[:3] for c in children]

    out = []
    out.append("// GENERATED by g1.cu_amd/csrc/gen_model_tables.py -- do not edit by hand.")
    out.append("// Unitree G1 model constants (MuJoCo 3.9.0 compilation of models/g1.xml + scene.xml,")
    out.append("// BSD-3 Unitree / MuJoCo Menagerie), read as data from the reference's generated header")
    out.append("// (reference: src/g1_model.h:5-474). MuJoCo dof/qpos ordering; quaternions (w,x,y,z).")
    out.append("// Free-joint qvel: [0:3] world linear, [3:6] body-local angular.")
    out.append("#pragma once\n")
    out.append("namespace g1 {\n")
    for k, v in idef.items():
        out.append(f"constexpr int {k} = {v};")
    out.append(f"constexpr int kMaxDepth = {max(depth)};")
    out.append(f"constexpr int kMaxEfc = 4 * kNFoot;   // pyramidal condim-3: 4 rows per contact")
    out.append(f"constexpr int kContactDofs = 12;        // free base (6) + one leg chain (6)\n")
    for ref, ours in INT_TABLES.items():
        vals = ints[ours]
        out.append(f"constexpr int {ours}[{len(vals)}] = {{{', '.join(map(str, vals))}}};")
    out.append("")
    out.append("// Derived topology (generator-checked): depth from the world body, and each body's")
    out.append("// children in DESCENDING index order (the order leaf->root sweeps accumulate them).")
    out.append(f"constexpr int body_depth[{nb}] = {{{', '.join(map(str, depth))}}};")
    out.append(f"constexpr int body_nchild[{nb}] = {{{', '.join(str(len(c)) for c in children)}}};")
    flat = [x for k in kids for x in k]
    out.append(f"constexpr int body_child[{nb * 3}] = {{{', '.join(map(str, flat))}}};\n")

    out.append("template <typename T> struct ModelT;\n")
    for dbl in (False, True):
        typ = "double" if dbl else "float"
        out.append(f"template <> struct ModelT<{typ}> {{")
        for ref, ours in FLOAT_DEFINES.items():
            out.append(f"  static constexpr {typ} {ours} = {flit(defines[ref], dbl)};")
        for ref, ours in FLOAT_TABLES.items():
            typ_, vals = arrays[ref]
            assert typ_ == "float"
            ncol = 4 if "quat" in ours else (3 if len(vals) % 3 == 0 and len(vals) >= 24 else 8)
            out.append(emit_float_table(ours, vals, dbl, ncol).rstrip("\n"))
        out.append("};\n")
    out.append("}  // namespace g1")
    with open(OUT, "w") as f:
        f.write("\n".join(out) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
