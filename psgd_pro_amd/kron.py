"""KronWhiten: the PSGD-Kron optimizer (dQ = Q^0.5 E Q^1.5, whitening preconditioner) on the HIP engine.

Drop-in for psgd_pro.KronWhiten / psgd_pro_fast.KronWhiten (psgd_pro.py:251-384, psgd_pro_fast.py:239-499): the same
constructor arguments, mutable attributes, step(closure) returning the closure's value and step_math(grads); plus
state_dict() / load_state_dict() (absent in the reference). Every parameter's preconditioner update and gradient
apply run through libpsgdk.so's grouped entry points (psgdk_kron2d_update / _apply / _balance,
psgdk_momentum_multi):
parameters of one shape and factor structure form a group of up to 16 that every kernel launch covers at once, and
no step synchronizes the host with the device.

Parameters are handled as m x n matrices after squeezing: 2-D as is, 1-D as 1 x n, scalars as 1 x 1 (one diagonal
factor). Tensors of order 3 or more are rejected (NotImplementedError).

Random draws (psgd_pro.py:123,35,59,138,345): draws="host" reproduces psgd_pro.py's stream on a CPU generator
(update coin, then per parameter the damping noise, two 32 x d starts per dense factor, the balancing coin) and
uploads the normals; draws="device" draws the coins on the CPU (update coin, then one balancing coin per parameter,
as psgd_pro_fast.py:482-483), then a 62-bit seed, and the library draws the step's normals on the GPU from it
(Philox4x32-10 and Box-Muller): psgdk_fill_normal fills the float32 buffer (the norm bounds' starts, float32 noise),
and bf16 noise is generated inside the grouped update's noise kernel (psgdk_kron2d_update_groups_drawn), the same
values as a filled bf16 buffer would hold.
"""
import collections
import contextlib
import ctypes

import torch

from . import _lib as L
from .ops import EagerOps

_K = L.NLB_K
# a parameter's noise generated inside the update: normals offset .. of the Philox sequence (seed, stream_id)
_Drawn = collections.namedtuple("_Drawn", "seed stream_id offset")


def _is_dense(size, numel, max_size, max_skew):
    # psgd_pro.py:189
    return not (size <= 1 or size > max_size or size ** 2 > max_skew * numel)


class _Lane:
    """A side stream (None: the caller's stream) with the workspaces of the groups it runs."""

    def __init__(self, stream, ws_upd, ws_app, ws_bal):
        self.stream, self.ws_upd, self.ws_app, self.ws_bal = stream, ws_upd, ws_app, ws_bal


class _Param:
    __slots__ = ("index", "shape", "m", "n", "kind", "Q", "P", "L", "group", "slot", "scalar")


class _Group:
    __slots__ = ("key", "members", "m", "n", "kind", "struct", "Qs", "Ps", "Ls", "Qt16", "P16", "g_dtype", "p_dtype")


class KronWhiten:
    """See the module docstring. Arguments as psgd_pro_fast.KronWhiten (psgd_pro_fast.py:245-264):

    ops: a plugin class from make_ops (EagerOps, the reference's default, is make_ops(())). The engine runs its own
      fused, grouped kernels rather than calling the plugin's methods one by one, and takes from the plugin what
      changes its arithmetic: the storage form of term1 and P (flags "tri" or "packed": the upper triangle only;
      "nan" poisons the lower triangle only in what the plugin's own methods return) and "bf16" (bf16 MFMA inputs).
      The kernel-selection flags (k1, k2, k2t, k2c, k2b, all) choose among the reference's CUDA/Triton/cuBLAS kernels
      and their size gates; here one HIP kernel set serves every size. A class that make_ops did not build raises
      TypeError, and a plugin asking for the Q-symmetrization in place of the Procrustes step (qsym) raises
      NotImplementedError.
    batch, cache_p, graph_rng, p2d: the reference's execution strategies for the same arithmetic (vmap over
      same-shape parameters, cached P, graph-captured draws, P kept as state). The engine always groups same-shape
      parameters, keeps P as state and can draw on the device (draws="device"), whatever these say; the reference's
      own checks on them (p2d with batch, cache_p with compile) are kept.
    compile: must be None (no torch.compile).

    Keyword-only extras: precision "fp32" | "bf16" (MFMA input precision of the contractions), draws "device" |
    "host", seed (a private CPU generator for the coins and host draws; None = torch's default generator, as the
    reference), tri (term1 and P kept as upper triangles), streams (side streams for the groups' update and apply
    chains; None: 3 for up to four groups, 4 for more, the faster count measured for each case), fuse_groups, and
    graphs, which must stay False: replaying the step from a captured HIP graph is switched off (a capture of the
    step aborted the process and the cause is not established)."""

    def __init__(self, params_with_grad,
                 preconditioner_max_size=float("inf"),
                 preconditioner_max_skew=1.0,
                 preconditioner_init_scale=None,
                 lr_params=0.001,
                 lr_preconditioner=0.1,
                 betaL=0.9,
                 damping=1e-9,
                 momentum=0.0,
                 grad_clip_max_amps=(2.0, 10.0),
                 preconditioner_update_probability=1.0,
                 update_preconditioner_first=True,
                 whiten_grad=True,
                 compile=None,
                 ops=EagerOps,
                 batch=False,
                 cache_p=False,
                 graph_rng=False,
                 p2d=False,
                 r2=False,
                 *,
                 precision=None,
                 draws="device",
                 seed=None,
                 tri=None,
                 streams=None,
                 graphs=False,
                 fuse_groups=True):
        self.lr_params = lr_params
        self.lr_preconditioner = lr_preconditioner
        self.betaL = betaL
        self.damping = damping
        self.momentum = momentum if (0 < momentum < 1) else 0.0
        self.grad_clip_max_amps = grad_clip_max_amps
        self.preconditioner_update_probability = preconditioner_update_probability
        self.update_preconditioner_first = update_preconditioner_first

        self._preconditioner_max_size = preconditioner_max_size
        self._preconditioner_max_skew = preconditioner_max_skew
        params_with_grad = [params_with_grad] if isinstance(params_with_grad, torch.Tensor) else params_with_grad
        self._params_with_grad = [p for p in params_with_grad if p.requires_grad]
        self._whiten_grad = whiten_grad
        if not whiten_grad:
            assert self.momentum > 0, "Cannot whiten momentum if the momentum setting is invalid."
        assert not (cache_p and compile is not None), "cache_p relies on tensor version counters: eager only"
        assert not (p2d and batch), "p2d keeps per-parameter P state; batch stacks parameters"
        if compile is not None:
            raise ValueError("compile: the HIP engine runs without torch.compile (pass compile=None)")
        if graphs:
            raise NotImplementedError(
                "graphs=True: replaying the step from a captured HIP graph is switched off. A capture of the step's "
                "device work (side streams forked inside torch.cuda.graph) aborted the process, and the cause is not "
                "established; the step runs its launches eagerly")
        self._r2 = bool(r2)  # procrustes_step_r2 (psgd_pro_fast.py:141-153) instead of procrustes_step2
        if ops is None:
            ops = EagerOps
        if not getattr(ops, "_psgdk", False):
            raise TypeError(f"ops: {getattr(ops, '__name__', ops)!r} was not built by psgd_pro_amd.make_ops; the "
                            "engine runs its own fused kernels and cannot call another plugin's methods")
        if getattr(ops, "qsym", False):
            raise NotImplementedError("ops.qsym: the Q-symmetrization in place of the Procrustes step is not built")
        flags = ops.flags
        self.ops = ops
        if precision is None:
            precision = "bf16" if "bf16" in flags else "fp32"
        if precision not in ("fp32", "bf16"):
            raise ValueError("precision: 'fp32' or 'bf16'")
        self._prec = L.PREC_BF16 if precision == "bf16" else L.PREC_F32
        self._tri = (3 if flags & {"tri", "packed"} else 0) if tri is None else (3 if tri else 0)
        if draws not in ("device", "host"):
            raise ValueError("draws: 'device' or 'host'")
        self._draws = draws
        self._gen = torch.Generator().manual_seed(seed) if seed is not None else None
        self.capture, self.pre = False, []
        self._params = None
        self._groups = None
        self._ms, self._counter_m = None, 0
        self._ws_upd, self._ws_app, self._ws_bal = L.Workspace(), L.Workspace(), L.Workspace()
        if streams is not None and int(streams) < 0:
            raise ValueError("streams: a count >= 0 or None")
        self._nstreams, self._lanes = (None if streams is None else int(streams)), None
        # one psgdk_kron2d_update_groups call for every bf16-path group: the factor work of all groups is batched
        # by factor side (the same operations as one call per group; larger launches may sum in another order)
        self._fuse = bool(fuse_groups)
        self._gev = {}  # per group: the event its update records when its factors are final
        self._overlap = True  # False: the whole update, then every balance, then every apply (each a fork / join)
        self._draw_in_update = True  # device draws: bf16 noise generated inside grouped updates (no noise buffer)
        self._draw_buf = self._draw_buf16 = None
        self._init_scale = preconditioner_init_scale
        if preconditioner_init_scale is not None:
            self._init([p.squeeze() for p in self._params_with_grad], preconditioner_init_scale)

    # ----------------------------------------------------------------------------------------------------------
    def _rand(self):
        return float(torch.rand([], generator=self._gen))

    def _init(self, grads, scale):
        """Factors of init_kron (psgd_pro.py:141-210): Q = scale^(1/order) I or ones, L = 0, and P = Q^T Q."""
        L.lib()
        self._params = []
        for i, g in enumerate(grads):
            if not g.is_cuda:
                raise RuntimeError("psgd_pro_amd.KronWhiten runs on the GPU; parameter %d is on %s" % (i, g.device))
            p = _Param()
            p.index, p.shape = i, tuple(g.shape)
            numel = max(1, g.numel())
            if g.dim() == 0:
                p.m, p.n, p.kind, p.scalar = 1, 1, (L.FACTOR_DIAG, L.FACTOR_NONE), True
            elif g.dim() == 1:
                d = g.shape[0]
                k = L.FACTOR_DENSE if _is_dense(d, numel, self._preconditioner_max_size,
                                                self._preconditioner_max_skew) else L.FACTOR_DIAG
                p.m, p.n, p.kind, p.scalar = 1, d, (L.FACTOR_NONE, k), False
            elif g.dim() == 2:
                m, n = g.shape
                k0 = L.FACTOR_DENSE if _is_dense(m, numel, self._preconditioner_max_size,
                                                 self._preconditioner_max_skew) else L.FACTOR_DIAG
                k1 = L.FACTOR_DENSE if _is_dense(n, numel, self._preconditioner_max_size,
                                                 self._preconditioner_max_skew) else L.FACTOR_DIAG
                p.m, p.n, p.kind, p.scalar = m, n, (k0, k1), False
            else:
                raise NotImplementedError(f"parameter {i}: tensors of order {g.dim()} are not supported")
            self._params.append(p)
        self._build_groups(grads, scale)

    def _build_groups(self, grads, scale):
        by_key = {}
        for p, g in zip(self._params, grads):
            prm = self._params_with_grad[p.index]
            key = (p.m, p.n, p.kind, g.dtype, prm.dtype, g.device)
            by_key.setdefault(key, []).append(p)
        self._groups = []
        for key, members in by_key.items():
            for c in range(0, len(members), L.MAXB):
                grp = _Group()
                grp.key, grp.members = key, members[c:c + L.MAXB]
                grp.m, grp.n, grp.kind = key[0], key[1], key[2]
                grp.g_dtype, grp.p_dtype = L.dtype_code(key[3]), L.dtype_code(key[4])
                dev = key[5]
                nb = len(grp.members)
                order = sum(k != L.FACTOR_NONE for k in grp.kind)
                grp.Qs, grp.Ps, grp.Ls = [None, None], [None, None], [None, None]
                grp.Qt16, grp.P16 = [None, None], [None, None]
                for f, (k, d) in enumerate(zip(grp.kind, (grp.m, grp.n))):
                    if k == L.FACTOR_NONE:
                        continue
                    s = scale if grp.members[0].scalar else scale ** (1.0 / order)
                    if k == L.FACTOR_DENSE:
                        Q = torch.eye(d, device=dev, dtype=torch.float32).mul_(s).expand(nb, d, d).contiguous()
                        P = torch.empty(nb, d, d, device=dev, dtype=torch.float32)
                        if (self._prec == L.PREC_BF16 and not self._tri and L.FACTOR_NONE not in grp.kind
                                and grp.m % 8 == 0 and grp.n % 8 == 0):
                            # bf16 shadows (Q^T and P) read by the bf16 contractions; the library keeps them current
                            grp.Qt16[f] = torch.empty(nb, d, d, device=dev, dtype=torch.bfloat16)
                            grp.P16[f] = torch.empty(nb, d, d, device=dev, dtype=torch.bfloat16)
                    else:
                        Q = torch.full((nb, d), s, device=dev, dtype=torch.float32)
                        P = torch.empty(nb, d, device=dev, dtype=torch.float32)
                    grp.Qs[f], grp.Ps[f] = Q, P
                    grp.Ls[f] = torch.zeros(nb, 1, device=dev, dtype=torch.float32)
                for j, p in enumerate(grp.members):
                    p.group, p.slot = grp, j
                grp.struct = self._struct(grp)
                self._groups.append(grp)
                self._refresh_p(grp)

    def _struct(self, grp):
        s = L.Kron2d()
        s.nb, s.prec, s.m, s.n = len(grp.members), self._prec, grp.m, grp.n
        s.kind[0], s.kind[1] = grp.kind
        s.g_dtype, s.p_dtype = grp.g_dtype, grp.p_dtype
        for f in range(2):
            if grp.Qs[f] is None:
                continue
            for j in range(len(grp.members)):
                s.Q[f][j] = grp.Qs[f][j].data_ptr()
                s.P[f][j] = grp.Ps[f][j].data_ptr()
                s.L[f][j] = grp.Ls[f][j].data_ptr()
                if grp.Qt16[f] is not None:
                    s.Qt16[f][j] = grp.Qt16[f][j].data_ptr()
                    s.P16[f][j] = grp.P16[f][j].data_ptr()
        return s

    def _refresh_p(self, grp):
        L.check(L.lib().psgdk_kron2d_refresh_p(grp.struct, 3, self._tri, L.stream_of(grp.Qs[0] if grp.Qs[0] is not None
                                                                                   else grp.Qs[1])))

    # ----------------------------------------------------------------------------------------------------------
    def _dense_dims(self, p):
        return [d for k, d in zip(p.kind, (p.m, p.n)) if k == L.FACTOR_DENSE]

    def _bind_sources(self, grp, srcs):
        """Points the group's G slots at this call's gradients (or momentum buffers) and sets their dtype."""
        s = grp.struct
        dt = srcs[grp.members[0].index].dtype
        for j, p in enumerate(grp.members):
            t = srcs[p.index]
            if t.dtype != dt:
                raise TypeError(f"parameters {grp.members[0].index} and {p.index} share a group but their gradients "
                                f"have dtypes {dt} and {t.dtype}")
            s.G[j] = t.data_ptr()
        s.g_dtype = L.dtype_code(dt)
        return dt

    def _draw_update(self, grads):
        """Normals of one update (noise, then per dense factor the SPD and skew starts) in psgd_pro.py's order;
        returns (per-parameter noise views, per-parameter V views, balance coins). The noise is drawn in the dtype
        of the tensor the update reads (the gradient, or the float32 momentum buffer when whiten_grad is off), as
        randn_like(G) does (psgd_pro_fast.py:200-206), the starts in float32 (the factors' dtype). Two persistent
        device buffers, one per dtype, each view at a multiple of 8 elements. With device draws, bf16 noise that only
        grouped updates read is not written to its buffer: its entries are _Drawn records (seed, stream id, offset
        in that buffer's layout), from which the update's noise kernel generates the same values."""
        ndt = [g.dtype if self._whiten_grad else torch.float32 for g in grads]
        r8 = lambda x: (x + 7) // 8 * 8
        lay, tot = [], {torch.float32: 0, torch.bfloat16: 0}  # per parameter: (noise offset, V offset, sizes)
        for p, dt in zip(self._params, ndt):
            a, b = p.m * p.n, sum(2 * _K * d for d in self._dense_dims(p))
            no = tot[dt]
            tot[dt] += r8(a)
            vo = tot[torch.float32]
            tot[torch.float32] += r8(b)
            lay.append((no, vo, a, b))
        dev = grads[0].device
        # device draws whose bf16 noise only grouped bf16-path updates read: that noise is generated inside the
        # update (psgdk_kron2d_update_groups_drawn, the same values) and the bf16 buffer is neither filled nor read
        fused_idx = {p.index for g in self._split_groups()[0] for p in g.members}
        drawn16 = self._draw_in_update and self._draws == "device" and tot[torch.bfloat16] > 0 and all(
            i in fused_idx for i, dt in enumerate(ndt) if dt == torch.bfloat16)
        bufs = {}
        for dt, attr in ((torch.float32, "_draw_buf"), (torch.bfloat16, "_draw_buf16")):
            if dt == torch.bfloat16 and drawn16:
                continue
            cur = getattr(self, attr, None)
            if cur is None or cur.numel() < max(1, tot[dt]):
                cur = torch.empty(max(1, tot[dt]), device=dev, dtype=dt)
                setattr(self, attr, cur)
            bufs[dt] = cur
        coins = []
        if self._draws == "host":
            host = {dt: torch.zeros(max(1, tot[dt]), dtype=dt) for dt in bufs}
            for p, dt, (no, vo, a, b) in zip(self._params, ndt, lay):
                host[dt][no:no + a] = torch.randn(a, generator=self._gen, dtype=dt)
                o = vo
                for d in self._dense_dims(p):
                    for _ in range(2):
                        host[torch.float32][o:o + _K * d] = torch.randn(_K * d, generator=self._gen)
                        o += _K * d
                coins.append(self._rand() < 0.01)
            for dt in bufs:
                if tot[dt]:
                    bufs[dt][:tot[dt]].copy_(host[dt][:tot[dt]].pin_memory(), non_blocking=True)
        else:
            # the normals from the library's counter-based generator (Philox4x32-10), keyed by a seed drawn from the
            # CPU generator after the coins: the step's whole draw is one launch per buffer, and the generator state
            # that state_dict saves determines it
            coins = (torch.rand(len(self._params), generator=self._gen) < 0.01).tolist()
            seed = int(torch.randint(0, 2 ** 62, (1,), generator=self._gen))
            st = L.stream_of(bufs[torch.float32])
            for sid, dt in enumerate((torch.float32, torch.bfloat16)):
                if tot[dt] and dt in bufs:
                    L.check(L.lib().psgdk_fill_normal(ctypes.c_void_p(bufs[dt].data_ptr()), tot[dt], L.dtype_code(dt),
                                                      seed, sid, st))
        noise, V = [], []
        for dt, (no, vo, a, b) in zip(ndt, lay):
            # stream id 1: the bf16 sequence (psgdk_fill_normal's stream_id of the bf16 buffer)
            noise.append(_Drawn(seed, 1, no) if dt not in bufs else bufs[dt][no:no + a])
            V.append(bufs[torch.float32][vo:vo + b] if b else None)
        return noise, V, coins

    # Groups share no state (each owns its factors, shadows and parameters), so their update and apply chains
    # run on side streams of default priority, each with its own workspaces: one group's memory-bound epilogues
    # and small kernels overlap another's GEMMs. The side streams start after the caller's stream reaches the
    # step and the caller's stream waits for all of them before it continues; results do not depend on the
    # number of streams.
    def side_streams(self):
        """The number of side streams the groups' chains use (streams=None: 3 for up to four groups, 4 for more;
        the runtime serves a process's streams from four hardware queues, and with few groups a fourth side stream
        only shares a queue (ViT-B, 4 groups: 10.36 against 10.39 ms/step), while many groups of small launches gain
        from it (the end-to-end ViT's 78 parameters: 1.51 against 1.69 ms per optimizer step))."""
        ng = len(self._groups) if self._groups else 0
        n = self._nstreams if self._nstreams is not None else (3 if ng <= 4 else 4)
        return 0 if ng < 2 else min(n, ng)

    def _lanes_for(self, dev):
        if self.side_streams() == 0:
            return [_Lane(None, self._ws_upd, self._ws_app, self._ws_bal)]
        if self._lanes is None or len(self._lanes) != self.side_streams():
            self._lanes = [_Lane(torch.cuda.Stream(device=dev), L.Workspace(), L.Workspace(), L.Workspace())
                           for _ in range(self.side_streams())]
        return self._lanes

    def _fork(self, dev):
        lanes = self._lanes_for(dev)
        cur = torch.cuda.current_stream(dev)
        for ln in lanes:
            if ln.stream is not None:
                ln.stream.wait_stream(cur)
        return cur, lanes

    @staticmethod
    def _join(cur, lanes):
        for ln in lanes:
            if ln.stream is not None:
                cur.wait_stream(ln.stream)

    @contextlib.contextmanager
    def _forked(self, dev):
        """The side streams forked from the caller's stream; joined back on leaving, also when a call raises."""
        cur, lanes = self._fork(dev)
        try:
            yield cur, lanes
        finally:
            self._join(cur, lanes)

    @staticmethod
    def _b16(grp):
        """The group takes the library's bf16 path (its b16_group rule): two factors, dense or diagonal with at least
        one dense, every dense factor with its bf16 shadows (bf16 precision, sides multiples of 8, full storage) and
        every operand under 2 GiB."""
        if L.FACTOR_NONE in grp.kind or L.FACTOR_DENSE not in grp.kind:
            return False
        for f, d in enumerate((grp.m, grp.n)):
            if grp.kind[f] == L.FACTOR_DENSE and (grp.Qt16[f] is None or d * d * 2 >= 2 ** 31):
                return False
        return grp.m * grp.n * 2 < 2 ** 31

    def _update_opts(self):
        return L.UpdateOpts(self.lr_preconditioner, self.betaL, self.damping, 0.0, self._tri, int(self._r2))

    def _apply_opts(self):
        max_avg, max_el = self.grad_clip_max_amps
        return L.ApplyOpts(self.lr_params, max_avg, max_el, self._tri)

    def _split_groups(self):
        """(the bf16-path groups one grouped update call takes, the groups updated one call each)"""
        fused = [g for g in self._groups if self._fuse and self._b16(g)][:L.MAX_GROUPS]
        return fused, [g for g in self._groups if not any(g is f for f in fused)]

    def _update_fused(self, fused, srcs, noise, V, ln, dev, events=None):
        """One grouped update of the bf16-path groups on the current stream (psgdk_kron2d_update_groups; with
        events, psgdk_kron2d_update_groups_ev, which records each group's event once its factors are final)."""
        o = self._update_opts()
        opts, nzs, vvs, drs = [], [], [], []
        for grp in fused:
            og = L.UpdateOpts(o.lr, o.betaL, o.damping, 0.0, o.tri, o.r2)
            og.grad_eps = torch.finfo(self._bind_sources(grp, srcs)).eps
            opts.append(og)
            nz = [noise[p.index] for p in grp.members]
            if isinstance(nz[0], _Drawn):  # a group's members share the gradient dtype, so all or none are drawn
                d = L.Draws(nz[0].seed, nz[0].stream_id)
                for b, x in enumerate(nz):
                    d.offset[b] = x.offset
                drs.append(ctypes.pointer(d))
                nzs.append(None)
            else:
                drs.append(None)
                nzs.append(L.ptrs(nz))
            vvs.append(L.ptrs([V[p.index] for p in grp.members]))
        ng = len(fused)
        garr = (ctypes.POINTER(L.Kron2d) * ng)(*[ctypes.pointer(g.struct) for g in fused])
        oarr = (ctypes.POINTER(L.UpdateOpts) * ng)(*[ctypes.pointer(x) for x in opts])
        narr = (ctypes.POINTER(ctypes.c_void_p) * ng)(*nzs)
        varr = (ctypes.POINTER(ctypes.c_void_p) * ng)(*vvs)
        st = L.stream_of(srcs[0])
        if any(d is not None for d in drs):
            darr = (ctypes.POINTER(L.Draws) * ng)(*drs)
            earr = L.ptrs([ev.cuda_event for ev in events]) if events is not None else None
            fn = L.lib().psgdk_kron2d_update_groups_drawn
            sz = ctypes.c_size_t(0)
            L.check(fn(ng, garr, oarr, narr, darr, varr, None, ctypes.byref(sz), st, earr))
            buf = ln.ws_upd.get(sz.value, dev)
            sz2 = ctypes.c_size_t(buf.numel())
            L.check(fn(ng, garr, oarr, narr, darr, varr, ctypes.c_void_p(buf.data_ptr()), ctypes.byref(sz2), st, earr))
            return
        if events is None:
            L.call_ws(L.lib().psgdk_kron2d_update_groups, ng, garr, oarr, narr, varr, ws=ln.ws_upd, device=dev,
                      stream=st)
            return
        earr = L.ptrs([ev.cuda_event for ev in events])
        fn = L.lib().psgdk_kron2d_update_groups_ev
        sz = ctypes.c_size_t(0)
        L.check(fn(ng, garr, oarr, narr, varr, None, ctypes.byref(sz), st, earr))
        buf = ln.ws_upd.get(sz.value, dev)
        sz2 = ctypes.c_size_t(buf.numel())
        L.check(fn(ng, garr, oarr, narr, varr, ctypes.c_void_p(buf.data_ptr()), ctypes.byref(sz2), st, earr))

    def _update_group(self, grp, srcs, noise, V, ln, dev):
        """One group's update on the current stream (psgdk_kron2d_update)."""
        o = self._update_opts()
        o.grad_eps = torch.finfo(self._bind_sources(grp, srcs)).eps
        nz = L.ptrs([noise[p.index] for p in grp.members])
        vv = L.ptrs([V[p.index] for p in grp.members])
        L.call_ws(L.lib().psgdk_kron2d_update, grp.struct, o, nz, vv, ws=ln.ws_upd, device=dev,
                  stream=L.stream_of(srcs[0]))

    def _balance_group(self, grp, coins, ln, dev):
        """psgd_pro.py:138-139 for the group's parameters whose coin came up, on the current stream."""
        flags = [int(coins[p.index]) for p in grp.members]
        if any(flags):
            fl = (ctypes.c_int32 * len(flags))(*flags)
            L.call_ws(L.lib().psgdk_kron2d_balance, grp.struct, fl, self._tri, ws=ln.ws_bal, device=dev,
                      stream=torch.cuda.current_stream(dev).cuda_stream)

    def _apply_group(self, grp, srcs, pre, ln, dev):
        """Precondition, clip and update the group's parameters on the current stream (psgdk_kron2d_apply)."""
        self._bind_sources(grp, srcs)
        prm = L.ptrs([self._params_with_grad[p.index] for p in grp.members])
        po = L.ptrs([pre[p.index] for p in grp.members]) if pre is not None else None
        L.call_ws(L.lib().psgdk_kron2d_apply, grp.struct, self._apply_opts(), prm, po, None, ws=ln.ws_app, device=dev,
                  stream=L.stream_of(srcs[0]))

    def _pre_buffers(self, dev):
        """The preconditioned gradients' outputs when `capture` is set (else None)."""
        if not self.capture:
            return None
        return [torch.empty(p.m, p.n, device=dev, dtype=torch.float32) for p in self._params]

    def _keep_pre(self, pre):
        if pre is not None:
            self.pre = [t.view(p.shape) for t, p in zip(pre, self._params)]

    @staticmethod
    def _on(ln, cur):
        return torch.cuda.stream(ln.stream if ln.stream is not None else cur)

    def _update(self, srcs, noise, V):
        dev = srcs[0].device
        with self._forked(dev) as (cur, lanes):
            fused, rest = self._split_groups()
            if fused:
                with self._on(lanes[0], cur):
                    self._update_fused(fused, srcs, noise, V, lanes[0], dev)
            for gi, grp in enumerate(rest):
                ln = lanes[(gi + (1 if fused else 0)) % len(lanes)]
                with self._on(ln, cur):
                    self._update_group(grp, srcs, noise, V, ln, dev)

    def _balance(self, coins, dev):
        """psgd_pro.py:138-139: balance the factors of every parameter whose coin came up (eager, rare)."""
        with self._forked(dev) as (cur, lanes):
            for gi, grp in enumerate(self._groups):
                ln = lanes[gi % len(lanes)]
                with self._on(ln, cur):
                    self._balance_group(grp, coins, ln, dev)

    def _apply(self, srcs):
        dev = srcs[0].device
        pre = self._pre_buffers(dev)
        with self._forked(dev) as (cur, lanes):
            for gi, grp in enumerate(self._groups):
                ln = lanes[gi % len(lanes)]
                with self._on(ln, cur):
                    self._apply_group(grp, srcs, pre, ln, dev)
        self._keep_pre(pre)

    def _group_event(self, grp):
        """A persistent event per group, created (recorded once) so that its handle exists for the library."""
        ev = self._gev.get(id(grp))
        if ev is None:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream())
            self._gev[id(grp)] = ev
        return ev

    def _update_then_apply(self, srcs, noise, V, coins, asrcs):
        """The update, then per group its balance (when one of its coins came up) and its apply, each group's after
        that group's own update only: the grouped update records a completion event per group
        (psgdk_kron2d_update_groups_ev), the groups updated one call each record theirs, and the balance and apply
        chains run on the side streams other than the grouped update's, smaller factor sides first (their batches
        end first). Each group goes through the same operations in the same order as with the whole update, then
        every balance, then every apply (bitwise the same results)."""
        dev = srcs[0].device
        pre = self._pre_buffers(dev)
        with self._forked(dev) as (cur, lanes):
            fused, rest = self._split_groups()
            done = {}
            if fused:
                evs = [self._group_event(g) for g in fused]
                with self._on(lanes[0], cur):
                    self._update_fused(fused, srcs, noise, V, lanes[0], dev, events=evs)
                done.update((id(g), ev) for g, ev in zip(fused, evs))
            for gi, grp in enumerate(rest):
                ln = lanes[(gi + (1 if fused else 0)) % len(lanes)]
                with self._on(ln, cur):
                    self._update_group(grp, srcs, noise, V, ln, dev)
                    ev = self._group_event(grp)
                    ev.record(ln.stream)
                    done[id(grp)] = ev
            # the grouped call joins all of its work into lanes[0]: the chains run on the other lanes
            alanes = lanes[1:] if fused else lanes
            side = lambda g: max(g.m if g.kind[0] == L.FACTOR_DENSE else 0, g.n if g.kind[1] == L.FACTOR_DENSE else 0)
            for i, grp in enumerate(sorted(self._groups, key=side)):
                ln = alanes[i % len(alanes)]
                with self._on(ln, cur):
                    ln.stream.wait_event(done[id(grp)])
                    self._balance_group(grp, coins, ln, dev)
                    self._apply_group(grp, asrcs, pre, ln, dev)
        self._keep_pre(pre)

    # ----------------------------------------------------------------------------------------------------------
    @torch.no_grad()
    def step_math(self, grads):
        """One step with the gradients given (psgd_pro_fast.py:441-490)."""
        grads = [g.squeeze() for g in grads]
        for i, (g, p) in enumerate(zip(grads, self._params_with_grad)):
            if g.dtype not in (torch.float32, torch.bfloat16):
                raise TypeError(f"gradient {i}: float32 or bfloat16 expected, got {g.dtype}")
            if g.device != p.device or not g.is_cuda:
                raise RuntimeError(f"gradient {i} is on {g.device}; its parameter is on {p.device} (GPU expected)")
            if g.numel() != p.numel():
                raise RuntimeError(f"gradient {i} has {g.numel()} elements, its parameter {p.numel()}")
        grads = [g if g.is_contiguous() else g.contiguous() for g in grads]
        if self._params is None:
            # psgd_pro.py:329-332: scale = (max_p mean|g|^4 + damping^4)^(-1/8) (one host read at initialisation)
            m4 = max(float(torch.mean(g.float().abs() ** 4)) for g in grads)
            self._init(grads, (m4 + self.damping ** 4) ** (-1.0 / 8))
        dev = grads[0].device
        beta = None
        if self.momentum > 0:
            beta = min(self._counter_m / (1 + self._counter_m), self.momentum)
            self._counter_m += 1
            if self._ms is None:
                self._ms = [torch.zeros(g.shape, device=g.device, dtype=torch.float32) for g in grads]
        else:
            self._ms, self._counter_m = None, 0
        update = self._rand() < self.preconditioner_update_probability
        noise = V = coins = None
        if update:
            noise, V, coins = self._draw_update(grads)
        # device work in segments; the balancing coins act between them, as in psgd_pro.py:138-139 (inside the
        # update, so before the apply when the update comes first)
        first = update and self.update_preconditioner_first
        if first and self._overlap and self.side_streams() >= 2:
            # each group's balance and apply start as soon as that group's own factors are final
            self._momentum_step(grads, beta)
            self._update_then_apply(grads if self._whiten_grad else self._ms, noise, V, coins,
                                    self._ms if self.momentum > 0 else grads)
            return
        self._device_work(grads, beta, first, not first, noise, V)
        if first and any(coins):
            self._balance(coins, dev)
        if first:
            self._device_work(grads, None, False, True, None, None)
        elif update:
            self._device_work(grads, None, True, False, noise, V)
            if any(coins):
                self._balance(coins, dev)

    def _momentum_step(self, grads, beta):
        """psgd_pro.py:340-341 on the caller's stream when beta is given: every parameter's momentum in one launch
        per 64 tensors."""
        if beta is None:
            return
        for c in range(0, len(grads), L.MAX_TENSORS):
            ch = range(c, min(c + L.MAX_TENSORS, len(grads)))
            numel = (ctypes.c_int64 * len(ch))(*[grads[i].numel() for i in ch])
            dts = (ctypes.c_int32 * len(ch))(*[L.dtype_code(grads[i].dtype) for i in ch])
            L.check(L.lib().psgdk_momentum_multi(len(ch), numel, beta, dts, L.ptrs([self._ms[i] for i in ch]),
                                                 L.ptrs([grads[i] for i in ch]), L.stream_of(grads[0])))

    def _device_work(self, grads, beta, do_update, do_apply, noise, V):
        """Momentum (when beta is given), preconditioner update, apply: kernel launches only."""
        self._momentum_step(grads, beta)
        src = grads if self._whiten_grad else self._ms
        if do_update and self.update_preconditioner_first:
            self._update(src, noise, V)
        if do_apply:
            self._apply(self._ms if self.momentum > 0 else grads)
        if do_update and not self.update_preconditioner_first:
            self._update(src, noise, V)

    @torch.no_grad()
    def step(self, closure):
        """psgd_pro.py:319-384: evaluates the closure, takes the gradients with torch.autograd.grad, steps, and
        returns whatever the closure returned."""
        with torch.enable_grad():
            closure_returns = closure()
            loss = closure_returns if isinstance(closure_returns, torch.Tensor) else closure_returns[0]
            grads = torch.autograd.grad(loss, self._params_with_grad)
        self.step_math(grads)
        return closure_returns

    # ----------------------------------------------------------------------------------------------------------
    def factors(self, i):
        """(Q, L) of parameter i as lists over its factors (views of the group storage; diagonal factors are
        vectors, a scalar parameter's factor is 0-d)."""
        p = self._params[i]
        Q, Ls = [], []
        for f in range(2):
            if p.kind[f] == L.FACTOR_NONE:
                continue
            q = p.group.Qs[f][p.slot]
            Q.append(q.view(()) if p.scalar else q)
            Ls.append(p.group.Ls[f][p.slot].view(()))
        return Q, Ls

    def state_dict(self):
        """Q, L (and P) per parameter, momentum buffers and counter, the CPU generator state and the mutable
        hyperparameters. P is saved for exactness of the next step; it is recomputed from Q when absent."""
        st = dict(version=1, hyper=dict(lr_params=self.lr_params, lr_preconditioner=self.lr_preconditioner,
                                        betaL=self.betaL, damping=self.damping, momentum=self.momentum,
                                        grad_clip_max_amps=tuple(self.grad_clip_max_amps),
                                        preconditioner_update_probability=self.preconditioner_update_probability,
                                        update_preconditioner_first=self.update_preconditioner_first),
                  counter_m=self._counter_m,
                  momentum_buffers=[m.clone() for m in self._ms] if self._ms is not None else None,
                  generator=self._gen.get_state() if self._gen is not None else None)
        if self._params is not None:
            for grp in self._groups:  # the bf16 path keeps only P's bf16 copy current between refreshes
                self._refresh_p(grp)
            st["params"] = []
            for p in self._params:
                ent = dict(shape=p.shape, kind=tuple(p.kind), Q=[], P=[], L=[])
                for f in range(2):
                    if p.kind[f] == L.FACTOR_NONE:
                        continue
                    ent["Q"].append(p.group.Qs[f][p.slot].clone())
                    ent["P"].append(p.group.Ps[f][p.slot].clone())
                    ent["L"].append(p.group.Ls[f][p.slot].clone())
                st["params"].append(ent)
        return st

    def load_state_dict(self, st):
        for k, v in st["hyper"].items():
            setattr(self, k, v)
        self._counter_m = st["counter_m"]
        saved = st["momentum_buffers"]
        if saved is None:
            self._ms = None
        elif self._ms is not None and [tuple(m.shape) for m in self._ms] == [tuple(m.shape) for m in saved]:
            for m, v in zip(self._ms, saved):  # into the existing buffers: their addresses stay valid
                m.copy_(v)
        else:
            dev = self._params_with_grad[0].device
            self._ms = [v.to(device=dev, dtype=torch.float32, copy=True) for v in saved]
        if st["generator"] is not None:
            if self._gen is None:
                self._gen = torch.Generator()
            self._gen.set_state(st["generator"])
        if "params" not in st:
            return
        dev = self._params_with_grad[0].device
        if self._params is None:
            grads = [torch.zeros(e["shape"], device=dev, dtype=p.dtype)
                     for e, p in zip(st["params"], self._params_with_grad)]
            self._init(grads, 1.0)
        for p, ent in zip(self._params, st["params"]):
            if tuple(ent["kind"]) != tuple(p.kind) or tuple(ent["shape"]) != p.shape:
                raise ValueError(f"state for parameter {p.index} does not match its shape/factor structure")
            fs = [f for f in range(2) if p.kind[f] != L.FACTOR_NONE]
            for j, f in enumerate(fs):
                p.group.Qs[f][p.slot].copy_(ent["Q"][j])
                p.group.Ls[f][p.slot].copy_(ent["L"][j])
                if ent.get("P"):
                    p.group.Ps[f][p.slot].copy_(ent["P"][j])
        have_p = all(ent.get("P") for ent in st["params"])
        for grp in self._groups:
            # bf16 shadows (Q^T, P) are derived state: rebuild them from the loaded Q (their fp32 P is what
            # state_dict saved, since it refreshes P first); other groups keep the saved P unless it is absent
            if not have_p or any(x is not None for x in grp.P16):
                self._refresh_p(grp)
