"""Sequential model of the reference's fused search kernel, traversal branch.

TEST INFRASTRUCTURE ONLY: it checks the C++ oracle (oracle/garfield_oracle.cpp)
on small inputs and nothing else uses it.

It is written from the reference kernel's own control flow,
select_path_contain_attr_filter_V2_without_output_with_post_pre_filter
(indexsearch/gpu_graph.cu:3266-3643, 4025-4130), as one block run one step at a
time: the shared arrays top_M_Cand / top_M_Cand_dis of TOPM + DEGREE entries
with the explored bit 0x80000000 in the id, merge_top's bisection
(gpu_graph.cu:162-222) and merge_top_with_recycle_list (:224-315) as written,
the visited set as a set of keys (the reference's 2048-slot table, which the
small inputs here never fill), and the 128 cross-edge slots of
work_mem_unsigned / work_mem_float.  Its structure is the reference's, not the
oracle's, so that a restatement mistake in either shows up as a difference.

Tie modes: tie=1 orders equal distances as the reference does -- comparisons
on distance alone and its sorting networks, warpSort (gpu_graph.cu:144-159)
and bitonic_sort_id_by_dis_no_explore (:77-101); tie=0 breaks distance ties by
cell-major position (the rule the oracle and the HIP kernels share), with
every sort a stable sort on that key.

Where the reference reads out of bounds, the model follows the oracle's
documented in-bounds rules: a cross slot i whose candidate i % 64 lies at or
beyond TOPM is empty (gpu_graph.cu:3572 tests TOPM < i % 64); the fallback scan
stops at the cell's size instead of 62500 (:3583); an empty entry's distance
is +inf (the reference leaves a stale value); entries are drawn below the first
cell's size.  The reference's INF_DIS (1e9) is +inf here.
"""
import numpy as np

SENT = 0xFFFFFFFF
EXPL = 0x80000000
IDM = 0x7FFFFFFF
ID30 = 0x3FFFFFFF
INF = float("inf")
MAX_ITER = 10000
HASH_RESET = 4
HASHLEN = 2048


def bitonic_no_explore(dis, ids, n):
    """bitonic_sort_id_by_dis_no_explore (gpu_graph.cu:77-101) on dis[:n], ids[:n]."""
    stride = 1
    while stride < n:
        step = stride
        while step > 0:
            for k in range(n // 2):
                a = 2 * step * (k // step)
                b = k % step
                u = a + step - 1 - b if step == stride else a + b
                d = a + b + step
                if d < n and dis[u] > dis[d]:
                    dis[u], dis[d] = dis[d], dis[u]
                    ids[u], ids[d] = ids[d], ids[u]
            step >>= 1
        stride <<= 1


def warp_sort(key, val, n):
    """warpSort (gpu_graph.cu:144-159) on n lanes: each round every lane reads
    its xor partner, then takes the partner's pair when the keys differ and
    the partner belongs on its side."""
    rng = 1
    while rng <= n:
        c = rng // 2
        while c >= 1:
            k1 = [key[l ^ c] if (l ^ c) < n else key[l] for l in range(n)]
            v1 = [val[l ^ c] if (l ^ c) < n else val[l] for l in range(n)]
            for l in range(n):
                p = bool(l & rng) == bool(l & c)
                if key[l] != k1[l] and ((key[l] < k1[l]) != p):
                    key[l], val[l] = k1[l], v1[l]
            c //= 2
        rng <<= 1


class KernelModel:
    def __init__(self, vectors, attrs, global_pid, P, cell_graphs, cross, tie=0):
        pid = [int(c) for c in global_pid]
        N = len(pid)
        self.P = P
        # get_idx_mapper (tools.cuh:862-915): cell starts, then each cell's
        # points in ascending point id
        size = [0] * P
        for c in pid:
            size[c] += 1
        self.seg = [0] * (P + 1)
        for c in range(P):
            self.seg[c + 1] = self.seg[c] + size[c]
        self.gidx = [0] * N
        self.lidx = [0] * N
        self.cell = pid
        fill = [0] * P
        for i, c in enumerate(pid):
            self.gidx[self.seg[c] + fill[c]] = i
            self.lidx[i] = fill[c]
            fill[c] += 1
        self.graph = np.ascontiguousarray(cell_graphs, np.int64)
        self.R = self.graph.shape[1]
        self.cross = np.ascontiguousarray(cross, np.int64)
        self.E = self.cross.shape[1] // P
        self.vec = np.ascontiguousarray(vectors, np.float64)
        self.attrs = np.ascontiguousarray(attrs, np.float64)
        self.tie = tie

    # ------------------------------------------------------------ order
    def _k(self, d, i):
        if self.tie == 1:
            return (d,)
        return (d, 0xFFFFFFFF if i == SENT else self.seg[self.cell[i & ID30]] + self.lidx[i & ID30])

    def le(self, d1, i1, d2, i2):
        return self._k(d1, i1) <= self._k(d2, i2)

    def lt(self, d1, i1, d2, i2):
        return self._k(d1, i1) < self._k(d2, i2)

    def sort_b(self, ids, dis, lo, n):
        """warpSort of entries [lo, lo + n) (tie 1) or a stable sort on the key."""
        k, v = dis[lo:lo + n], ids[lo:lo + n]
        if self.tie == 1:
            warp_sort(k, v, n)
        else:
            order = sorted(range(n), key=lambda t: self._k(k[t], v[t]))
            k, v = [k[t] for t in order], [v[t] for t in order]
        dis[lo:lo + n], ids[lo:lo + n] = k, v

    def sort_net(self, ids, dis, n):
        if self.tie == 1:
            bitonic_no_explore(dis, ids, n)
        else:
            order = sorted(range(n), key=lambda t: self._k(dis[t], ids[t]))
            ids[:n], dis[:n] = [ids[t] for t in order], [dis[t] for t in order]

    def _ranks(self, a_id, a_d, n, b_id, b_d, m):
        """merge_top's destination of every entry (gpu_graph.cu:172-206): the
        bisection over the other list as written, then the own index."""
        out = []
        for i in range(n):
            v = (a_d[i], a_id[i])
            r, tmp = 0, m
            while tmp > 1:
                half = tmp // 2
                if self.le(b_d[r + half], b_id[r + half], *v):
                    r += half
                tmp -= half
            r += 1 if self.le(b_d[r], b_id[r], *v) else 0
            out.append(r + i)
        for j in range(m):
            v = (b_d[j], b_id[j])
            r, tmp = 0, n
            while tmp > 1:
                half = tmp // 2
                if self.lt(a_d[r + half], a_id[r + half], *v):
                    r += half
                tmp -= half
            r += 1 if self.lt(a_d[r], a_id[r], *v) else 0
            out.append(r + j)
        return out

    def merge_top(self, a_id, a_d, b_id, b_d):
        """merge_top (gpu_graph.cu:162-222) on two lists, in place."""
        n, m = len(a_id), len(b_id)
        pos = self._ranks(a_id, a_d, n, b_id, b_d, m)
        vals = [(a_id[i], a_d[i]) for i in range(n)] + [(b_id[j], b_d[j]) for j in range(m)]
        for p, (i, d) in zip(pos, vals):
            if p < n:
                a_id[p], a_d[p] = i, d
            elif p < n + m:
                b_id[p - n], b_d[p - n] = i, d

    # ------------------------------------------------------------ search
    def _dist(self, q, g):
        t = self.vec[g] - q
        return float(np.dot(t, t))

    def _passes(self, g, lo, hi):
        a = self.attrs[g]
        return bool(np.all((a >= lo) & (a <= hi)))

    def search(self, q, lo, hi, cells, entry, L, K=10, rl=10, max_iter=MAX_ITER):
        """One traversal query over the ordered cells; returns (ids, dists,
        expansions, distance evaluations, expanded point ids, recycle list)."""
        R, E, P = self.R, self.E, self.P
        q = np.asarray(q, np.float64)
        lo = np.asarray(lo, np.float64)
        hi = np.asarray(hi, np.float64)
        top = [SENT] * (L + R)
        dis = [INF] * (L + R)
        rec_id = [SENT] * rl
        rec_d = [INF] * rl
        H = set()
        nexp = ndist = 0
        expanded = []

        def merge_with_recycle():
            # merge_top_with_recycle_list (gpu_graph.cu:224-315); the ranks
            # are a permutation of [0, L + R), so every entry is rewritten
            newt = [SENT] * (L + R)
            newd = [INF] * (L + R)
            pos = self._ranks(top, dis, L, top[L:], dis[L:], R)
            vals = [(top[i], dis[i]) for i in range(L + R)]
            for k, (p, (i, d)) in enumerate(zip(pos, vals)):
                if p >= L:
                    if k < L and i != SENT:
                        if not self._passes(i & 0x3FFFFFFF, lo, hi):
                            i, d = SENT, INF
                    elif k >= L:
                        i, d = SENT, INF
                if p < L + R:
                    newt[p], newd[p] = i, d
            top[:], dis[:] = newt, newd

        def evict_to_recycle():
            # gpu_graph.cu:3412-3425 / 3536-3546
            self.sort_b(top, dis, L, R)
            if top[L] != SENT:
                b_id, b_d = top[L:], dis[L:]
                self.merge_top(rec_id, rec_d, b_id, b_d)
                top[L:], dis[L:] = b_id, b_d

        for i in range(R):
            top[L + i] = self.gidx[self.seg[cells[0]] + int(entry[i])]
            H.add(top[L + i])           # the entry's point id (gpu_graph.cu:3349)
        for p_i, pid in enumerate(cells):
            base = self.seg[pid]
            for i in range(R):
                if top[L + i] == SENT:
                    dis[L + i] = INF
                    continue
                dis[L + i] = self._dist(q, top[L + i])
                if p_i == 0:
                    ndist += 1
            self.sort_b(top, dis, L, R)
            merge_with_recycle()
            evict_to_recycle()
            for it in range(max_iter):
                if (it + 1) % HASH_RESET == 0:
                    H = set(self.lidx[t & IDM] for t in top if t != SENT)
                assert len(H) < HASHLEN
                to_explore = SENT
                for j in range(L):
                    if (top[j] & EXPL) == 0:
                        to_explore = self.lidx[top[j]]
                        expanded.append(top[j])
                        top[j] |= EXPL
                        break
                if to_explore == SENT:
                    break
                nexp += 1
                for j in range(R):
                    nl = int(self.graph[base + to_explore, j])
                    g = self.gidx[base + nl]
                    if nl in H:
                        dis[L + j] = INF
                    else:
                        H.add(nl)
                        dis[L + j] = self._dist(q, g)
                        ndist += 1
                    top[L + j] = g
                self.sort_b(top, dis, L, R)
                if top[L] != SENT:
                    merge_with_recycle()
                    evict_to_recycle()
            for i in range(L):
                top[i] |= EXPL
            H = set()
            if p_i < len(cells) - 1:
                nxt = cells[p_i + 1]
                nbase, nsz = self.seg[nxt], self.seg[nxt + 1] - self.seg[nxt]
                wid = [SENT] * 128
                wd = [INF] * 128
                for i in range(128):
                    ci = i % 64
                    if ci >= L or top[ci] == SENT:
                        continue
                    pure = top[ci] & IDM
                    j = 0
                    while j < E:
                        nl = int(self.cross[pure, nxt * E + j])
                        j += 1
                        if nl not in H:
                            H.add(nl)
                            wid[i] = self.gidx[nbase + nl]
                            break
                        if j == E:
                            for rp in range(min(62500, nsz)):
                                if rp not in H:
                                    H.add(rp)
                                    wid[i] = self.gidx[nbase + rp]
                                    break
                for i in range(128):
                    if wid[i] != SENT:
                        wd[i] = self._dist(q, wid[i])
                        ndist += 1
                self.sort_net(wid, wd, 128)
                H = set()
                for i in range(R):
                    top[L + i] = wid[i]
                    if wid[i] != SENT:
                        H.add(self.lidx[wid[i]])
                for i in range(128 - R):
                    if wid[R + i] != SENT:
                        H.add(self.lidx[wid[R + i]])
                a_id, a_d = top[:L], dis[:L]
                b_id, b_d = wid[R:R + 64], wd[R:R + 64]
                self.merge_top(a_id, a_d, b_id, b_d)
                top[:L], dis[:L] = a_id, a_d
            for i in range(L):
                if top[i] != SENT:
                    H.add(self.lidx[top[i] & IDM])
        # post-filter, sort, recycle merge (gpu_graph.cu:4025-4047)
        for i in range(L):
            if top[i] != SENT and not self._passes(top[i] & IDM, lo, hi):
                top[i], dis[i] = SENT, INF
        a_id, a_d = top[:L], dis[:L]
        self.sort_net(a_id, a_d, L)
        recycle = list(zip(rec_id, rec_d))
        if rec_id[0] != SENT:
            self.merge_top(a_id, a_d, list(rec_id), list(rec_d))
        ids, dists = [], []
        for i, d in zip(a_id, a_d):
            if len(ids) == K:
                break
            if i == SENT or (i & IDM) in ids:
                continue
            ids.append(i & IDM)
            dists.append(d)
        while len(ids) < K:
            ids.append(0x7FFFFFFF)
            dists.append(INF)
        return ids, dists, nexp, ndist, [e & IDM for e in expanded], recycle

    # ------------------------------------------------------- full graph
    def full_graph(self, FE):
        """assemble_edges (full_graph_search.cuh:984-997): for point b and
        every cell pid in order, FE edges -- the own cell's graph row when pid
        is b's cell, else b's cross edges into pid -- mapped to point ids
        (local ids reduced modulo the cell size, the oracle's in-bounds rule;
        an empty cell gives 0xFFFFFFFF)."""
        N, P = len(self.cell), self.P
        out = np.full((N, FE * P), SENT, np.uint32)
        for b in range(N):
            for i in range(FE * P):
                pid, eid = i // FE, i % FE
                sz = self.seg[pid + 1] - self.seg[pid]
                if sz == 0:
                    continue
                if self.cell[b] == pid:
                    v = int(self.graph[self.seg[pid] + self.lidx[b], eid])
                else:
                    v = int(self.cross[b, pid * self.E + eid])
                out[b, i] = self.gidx[self.seg[pid] + v % sz]
        return out

    def search_full(self, q, lo, hi, fgraph, fentry, L, K=10, max_iter=MAX_ITER):
        """The full-graph branch (gpu_graph.cu:3644-3787) and the common
        post-filter (:4025-4047) for one query; returns (ids, dists,
        expansions, distance evaluations, expanded point ids)."""
        BD = fgraph.shape[1]
        q = np.asarray(q, np.float64)
        lo = np.asarray(lo, np.float64)
        hi = np.asarray(hi, np.float64)
        top = [SENT] * (L + BD)
        dis = [INF] * (L + BD)
        nexp = ndist = 0
        expanded = []
        H = set()
        for i in range(BD):
            top[L + i] = int(fentry[i])
            H.add(top[L + i])
        for j in range(BD):
            dis[L + j] = self._dist(q, top[L + j])
            ndist += 1

        def sort_and_merge():
            b_id, b_d = top[L:], dis[L:]
            self.sort_net(b_id, b_d, BD)
            a_id, a_d = top[:L], dis[:L]
            self.merge_top(a_id, a_d, b_id, b_d)
            top[:L], dis[:L] = a_id, a_d
            top[L:], dis[L:] = b_id, b_d

        sort_and_merge()
        for it in range(max_iter):
            if (it + 1) % HASH_RESET == 0:
                H = set(t & IDM for t in top if t != SENT)
            assert len(H) < HASHLEN
            to_explore = SENT
            for j in range(L):
                if (top[j] & EXPL) == 0:
                    to_explore = top[j]
                    top[j] |= EXPL
                    break
            if to_explore == SENT:
                break
            nexp += 1
            expanded.append(to_explore)
            for j in range(BD):
                g = int(fgraph[to_explore, j])
                if g == SENT or g in H:
                    top[L + j], dis[L + j] = SENT, INF
                else:
                    H.add(g)
                    top[L + j], dis[L + j] = g, self._dist(q, g)
                    ndist += 1
            sort_and_merge()
        for i in range(L):
            if top[i] != SENT and not self._passes(top[i] & IDM, lo, hi):
                top[i], dis[i] = SENT, INF
        a_id, a_d = top[:L], dis[:L]
        self.sort_net(a_id, a_d, L)
        ids, dists = [], []
        for i, d in zip(a_id, a_d):
            if len(ids) == K:
                break
            if i == SENT or (i & IDM) in ids:
                continue
            ids.append(i & IDM)
            dists.append(d)
        while len(ids) < K:
            ids.append(0x7FFFFFFF)
            dists.append(INF)
        return ids, dists, nexp, ndist, expanded

    # ------------------------------------------------------- dual channel
    def _merge_recycle_n(self, top, dis, L, n, lo, hi):
        """merge_top_with_recycle_list (gpu_graph.cu:224-315) of the n entries
        after top[:L] into top[:L]: list entries pushed out keep their place
        in the tail only if they pass the filter; tail entries pushed out
        become empty."""
        newt = [SENT] * (L + n)
        newd = [INF] * (L + n)
        pos = self._ranks(top[:L], dis[:L], L, top[L:L + n], dis[L:L + n], n)
        for k in range(L + n):
            i, d, p = top[k], dis[k], pos[k]
            if p >= L:
                if k < L and i != SENT:
                    if not self._passes(i & ID30, lo, hi):
                        i, d = SENT, INF
                elif k >= L:
                    i, d = SENT, INF
            newt[p], newd[p] = i, d
        top[:L + n], dis[:L + n] = newt, newd

    def search_dual(self, q, lo, hi, cells, entry, L, K=10, rl=10, max_iter=MAX_ITER):
        """Traversal of select_path_contain_attr_filter_V2_without_output_
        dual_channel_in_turn_with_prefilter (gpu_graph.cu:6249-6640) for one
        query whose cells are not all little: top_M_Cand of TOPM + 2 DEGREE
        entries, explored bits 31 (channel 0) and 30 (channel 1) in the id,
        the visited set of point ids, `turn` and `main_channel` as in the
        kernel.  In-bounds rules: entry[i] is reduced modulo its cell's size;
        cross-edge indexes at or beyond E are skipped (the reference reads 2
        edges per partner and per switch slot); equal keys met in one step
        enter the visited set in slot order.  Returns (ids, dists,
        expansions, distance evaluations, filled switch slots)."""
        R, E = self.R, self.E
        R2 = 2 * R
        q = np.asarray(q, np.float64)
        lo = np.asarray(lo, np.float64)
        hi = np.asarray(hi, np.float64)
        top = [SENT] * (L + R2)
        dis = [INF] * (L + R2)
        rec_id = [SENT] * rl
        rec_d = [INF] * rl
        H = set()
        nexp = ndist = nslot = 0
        psize = len(cells)
        size = lambda c: self.seg[c + 1] - self.seg[c]
        gid = lambda c, l: self.gidx[self.seg[c] + l]
        pid = [cells[0], cells[1] if psize >= 2 else cells[0]]
        L2 = (L + 1) // 2
        for i in range(L):
            mask = 0 if pid[0] == pid[1] else 1 << (30 + i // L2)
            c = pid[i // L2]
            top[i] = gid(c, int(entry[i]) % size(c)) | mask
            H.add(top[i] & ID30)
        cur = 2 if psize >= 2 else 1
        main_channel = 0
        turn = 0
        for i in range(L):
            if top[i] != SENT:
                dis[i] = self._dist(q, top[i] & ID30)
                ndist += 1
        a_id, a_d = top[:L], dis[:L]
        self.sort_net(a_id, a_d, L)
        top[:L], dis[:L] = a_id, a_d
        for epoch in range(max_iter):
            if (epoch + 1) % HASH_RESET == 0:
                H = set(t & ID30 for t in top[:L + R2] if t != SENT)
            assert len(H) < HASHLEN
            to_explore = [SENT, SENT]
            shift = 31 - main_channel if pid[0] == pid[1] else 31 - turn
            mask = 1 << shift
            for j in range(L):
                if (top[j] & mask) == 0:
                    to_explore[turn] = self.lidx[top[j] & ID30]
                    top[j] |= mask
                    break
            if to_explore[turn] != SENT:
                g = gid(pid[turn], to_explore[turn])
                for j in range(min(2, E)):
                    v = int(self.cross[g, pid[turn ^ 1] * E + j])
                    if v not in H:               # hash_peek of the local id's value
                        to_explore[turn ^ 1] = v
                        break
            if to_explore[turn] == SENT:
                if cur == psize and pid[0] == pid[1]:
                    break
                if cur == psize:
                    pid[turn] = pid[turn ^ 1]
                    main_channel = turn ^ 1
                    continue
                next_pid = cells[cur]
                mask = 1 << (30 + turn)
                wid = [SENT] * 128
                wd = [INF] * 128
                for i in range(128):
                    if i % 64 >= L or top[i % 64] == SENT or i // 64 >= E:
                        continue
                    nl = int(self.cross[top[i % 64] & ID30, next_pid * E + i // 64])
                    ng = gid(next_pid, nl)
                    if ng not in H:
                        H.add(ng)
                        wid[i], wd[i] = ng | mask, 0.0
                        nslot += 1
                for i in range(128):
                    if wid[i] != SENT:
                        wd[i] = self._dist(q, wid[i] & ID30)
                        ndist += 1
                self.sort_net(wid, wd, 128)
                t2, d2 = top[:L] + wid, dis[:L] + wd
                self._merge_recycle_n(t2, d2, L, 128, lo, hi)
                top[:L], dis[:L] = t2[:L], d2[:L]
                wid, wd = t2[L:], d2[L:]
                self.sort_net(wid, wd, 128)
                if wid[0] != SENT:
                    self.merge_top(rec_id, rec_d, wid, wd)
                pid[turn] = next_pid
                cur += 1
                continue
            for ch in (0, 1):
                base = L + ch * R
                if to_explore[ch] == SENT:
                    for i in range(R):
                        top[base + i], dis[base + i] = SENT, INF
                    continue
                nexp += 1
                mask = 0 if pid[0] == pid[1] else 1 << (30 + ch)
                for j in range(R - (0 if ch == turn else 1)):
                    local = int(self.graph[self.seg[pid[ch]] + to_explore[ch], j])
                    g = gid(pid[ch], local)
                    if g in H:
                        top[base + j], dis[base + j] = SENT, INF
                    else:
                        H.add(g)
                        top[base + j], dis[base + j] = g | mask, 0.0
                if ch != turn:
                    g = gid(pid[ch], to_explore[ch])
                    if g in H:
                        top[base + R - 1], dis[base + R - 1] = SENT, INF
                    else:
                        H.add(g)
                        top[base + R - 1], dis[base + R - 1] = g | mask, 0.0
            turn ^= 1
            for i in range(L, L + R2):
                if top[i] != SENT:
                    dis[i] = self._dist(q, top[i] & ID30)
                    ndist += 1
            self.sort_b(top, dis, L, R2)
            if top[L] != SENT:
                self._merge_recycle_n(top, dis, L, R2, lo, hi)
                self.sort_b(top, dis, L, R2)
                if top[L] != SENT:
                    b_id, b_d = top[L:], dis[L:]
                    self.merge_top(rec_id, rec_d, b_id, b_d)
                    top[L:], dis[L:] = b_id, b_d
        for i in range(L):
            if top[i] != SENT and not self._passes(top[i] & ID30, lo, hi):
                top[i], dis[i] = SENT, INF
        a_id, a_d = top[:L], dis[:L]
        self.sort_net(a_id, a_d, L)
        if rec_id[0] != SENT:
            self.merge_top(a_id, a_d, list(rec_id), list(rec_d))
        ids, dists = [], []
        for i, d in zip(a_id, a_d):
            if len(ids) == K:
                break
            if i == SENT or (i & ID30) in ids:
                continue
            ids.append(i & ID30)
            dists.append(d)
        while len(ids) < K:
            ids.append(0x7FFFFFFF)
            dists.append(INF)
        return ids, dists, nexp, ndist, nslot
