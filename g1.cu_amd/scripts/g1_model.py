"""Model constants for host-side Python (state generation, checks), read from the generated
table header g1.cu_amd/csrc/g1_model_tables.h so there is a single source of truth."""
import os
import re

import numpy as np

_HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "csrc", "g1_model_tables.h")

NBODY, NQ, NV, NU, NFOOT = 31, 36, 35, 29, 8
OBS_DIM, ACT_DIM = 100, 29


def _parse():
    text = open(_HDR).read()
    ints = {m.group(1): np.array([int(v) for v in m.group(3).split(",")], np.int64)
            for m in re.finditer(r"constexpr int (\w+)\[(\d+)\] = \{([^}]*)\};", text)}
    body_f = text.split("template <> struct ModelT<float> {")[1].split("};\n\ntemplate")[0]
    body_d = text.split("template <> struct ModelT<double> {")[1].split("};\n\n}")[0]

    def floats(body, suffix):
        out = {}
        for m in re.finditer(r"static constexpr \w+ (\w+)\[(\d+)\] = \{([^}]*)\};", body, re.S):
            vals = [v.strip().rstrip("f") for v in m.group(3).replace("\n", " ").split(",") if v.strip()]
            out[m.group(1)] = np.array([float(v) for v in vals], np.float64)
        for m in re.finditer(r"static constexpr \w+ (\w+) = ([^;]+);", body):
            out[m.group(1)] = float(m.group(2).rstrip("f"))
        return out

    return ints, floats(body_f, "f"), floats(body_d, "")


INTS, _F32, _F64 = _parse()


def table(name, dtype=np.float32):
    """A model table as float32 (the device literals) or float64."""
    src = _F32 if np.dtype(dtype) == np.float32 else _F64
    v = src[name]
    return np.asarray(v, dtype=dtype) if np.ndim(v) else dtype(v)


qpos_stand = table("qpos_stand")
act_frc_hi = table("act_frc_hi")
act_frc_lo = table("act_frc_lo")
act_kd = table("act_kd")
act_kp = table("act_kp")
act_ctrl_lo = table("act_ctrl_lo")
act_ctrl_hi = table("act_ctrl_hi")
foot_lpos = table("foot_lpos").reshape(NFOOT, 3)
foot_radius = table("foot_radius")
dt = table("dt")
