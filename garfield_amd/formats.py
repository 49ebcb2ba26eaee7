"""Readers and writers of the GMG index files and driver inputs (numpy).

Byte layouts follow the reference's writers and readers (all little-endian,
32-bit fields):
  .fvecs            per row i32 dim + dim f32            (tools.cuh:85-106)
  per-cell graph    i32 n, i32 R, n*R u32 local ids       (indexbuild/cagra_build.py:121-127)
  cross-cell graph  i32 N, i32 P*E, N*(P*E) u32 local ids (indexbuild/global_graph_build.py:167-176)
  grid              i32 N, i32 a, i32 g[a]; per attribute l_q[g], r_q[g], pid[N];
                    then global_pid[N]                    (indexbuild/tools.py:127-141)
  attrs             u32 N, u32 a, N*a i32                 (tools.cuh:746-765)
  ranges            Q*a*(i32 lo, i32 hi), no header       (tools.cuh:274-291)
  ground truth      u32 Q, u32 K, Q*K u32                 (tools.cuh:804-834)
  cluster labels    i32 N, N*i32                          (indexbuild/clustering.py:84-87)
"""
import numpy as np


def write_fvecs(path, x):
    x = np.ascontiguousarray(x, np.float32)
    n, d = x.shape
    rows = np.empty((n, d + 1), np.float32)
    rows[:, 0] = np.array([d], np.int32).view(np.float32)[0]
    rows[:, 1:] = x
    rows.tofile(path)


def read_fvecs(path):
    raw = np.fromfile(path, np.int32)
    if raw.size == 0:
        raise ValueError(f"empty fvecs {path}")
    d = int(raw[0])
    if d <= 0 or raw.size % (d + 1):
        raise ValueError(f"bad fvecs {path}")
    rows = raw.reshape(-1, d + 1)
    if np.any(rows[:, 0] != d):
        raise ValueError(f"inconsistent dimension in {path}")
    return rows[:, 1:].view(np.float32).copy()


def write_graph(path, g):
    g = np.ascontiguousarray(g, np.uint32)
    with open(path, "wb") as f:
        f.write(np.array([g.shape[0], g.shape[1]], np.int32).tobytes())
        f.write(g.tobytes())


def read_graph(path):
    raw = np.fromfile(path, np.uint32)
    n, k = int(raw[0]), int(raw[1])
    if raw.size != 2 + n * k:
        raise ValueError(f"graph size mismatch in {path}")
    return raw[2:].reshape(n, k).copy()


def write_grid(path, grid, l_q, r_q, pid_lists, global_pid):
    grid = np.asarray(grid, np.int32)
    n = len(global_pid)
    with open(path, "wb") as f:
        f.write(np.array([n, len(grid)], np.int32).tobytes())
        f.write(grid.tobytes())
        for lq, rq, pl in zip(l_q, r_q, pid_lists):
            f.write(np.asarray(lq, np.int32).tobytes())
            f.write(np.asarray(rq, np.int32).tobytes())
            f.write(np.asarray(pl, np.int32).tobytes())
        f.write(np.asarray(global_pid, np.int32).tobytes())


def read_grid(path):
    raw = np.fromfile(path, np.int32)
    n, a = int(raw[0]), int(raw[1])
    grid = raw[2:2 + a].copy()
    pos = 2 + a
    l_q, r_q, pids = [], [], []
    for d in range(a):
        g = int(grid[d])
        l_q.append(raw[pos:pos + g].copy()); pos += g
        r_q.append(raw[pos:pos + g].copy()); pos += g
        pids.append(raw[pos:pos + n].copy()); pos += n
    global_pid = raw[pos:pos + n].copy()
    if pos + n != raw.size:
        raise ValueError(f"grid size mismatch in {path}")
    return grid, l_q, r_q, pids, global_pid


def write_attrs(path, attrs):
    attrs = np.ascontiguousarray(attrs, np.int32)
    with open(path, "wb") as f:
        f.write(np.array(attrs.shape, np.uint32).tobytes())
        f.write(attrs.tobytes())


def read_attrs(path):
    raw = np.fromfile(path, np.int32)
    n, a = int(raw[0]), int(raw[1])
    if raw.size != 2 + n * a:
        raise ValueError(f"attrs size mismatch in {path}")
    return raw[2:].reshape(n, a).copy()


def write_ranges(path, lo, hi):
    lo = np.asarray(lo, np.int32)
    hi = np.asarray(hi, np.int32)
    np.stack([lo, hi], axis=2).astype(np.int32).tofile(path)


def read_ranges(path, a):
    raw = np.fromfile(path, np.int32).reshape(-1, a, 2)
    return raw[:, :, 0].copy(), raw[:, :, 1].copy()


def write_gt(path, gt):
    gt = np.ascontiguousarray(gt, np.uint32)
    with open(path, "wb") as f:
        f.write(np.array(gt.shape, np.uint32).tobytes())
        f.write(gt.tobytes())


def read_gt(path):
    raw = np.fromfile(path, np.uint32)
    q, k = int(raw[0]), int(raw[1])
    return raw[2:2 + q * k].reshape(q, k).copy()


def write_labels(path, labels):
    labels = np.asarray(labels, np.int32)
    with open(path, "wb") as f:
        f.write(np.array([labels.size], np.int32).tobytes())
        f.write(labels.tobytes())


def read_labels(path):
    raw = np.fromfile(path, np.int32)
    n = int(raw[0])
    return raw[1:1 + n].copy()
