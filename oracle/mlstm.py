"""CPU oracle for the mLSTM kernels: test infrastructure, not product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for
``cpu_baseline``, as the timed CPU path).  The product path
(``xlstm_hip``) never calls it and fails loudly when its HIP library is
missing.

Every function restates, in torch-on-CPU code written for this repository,
the torch-native algorithm of MLXPorts/xLSTM-metal (paths relative to the
reference root; ``VTN`` = ``kernel_development/xlstm/mlstm_block/
mlstm_chunkwise/vendored/torch/native``, ``REC`` = ``kernel_development/
xlstm/mlstm_block/mlstm_recurrent/recurrent``, ``PV`` =
``kernel_development/xlstm/mlstm_block/mslstm_parallel/vendored``, ``PT`` =
``kernel_development/xlstm/mlstm_block/mslstm_parallel/torch``).  The order
of operations and the dtype of every intermediate follow the reference so
that, run in float32 on the CPU, results match it to rounding.

How each function is pinned (tests/test_oracle_*.py):

* ``mlstm_chunkwise`` / ``mlstm_chunkwise_fw``: equals the recurrent
  sequence loop in float64 (exact identity of the two formulations, with and
  without initial states); is invariant to the chunk size; equals the
  quadratic parallel form (``mlstm_parallel_fw``) and a stabiliser-free
  brute-force O(S^2) closed form; single-token closed form; q = 0 gives
  h = 0.
* ``mlstm_recurrent_step`` / ``mlstm_recurrent_sequence``: equal the
  independent numpy restatement ``oracle.canonical_np`` (which follows the
  reference's own parity helper ``tests/parity/canonical_reference.py``),
  the gate known-answer values of ``tests/test_mlx_torch_numerical_parity.py``
  and the committed float64 fixtures under ``tests/golden``.
* ``mlstm_parallel_fw``: equals the brute-force closed form.
* ``mlstm_recurrent_kernel_cell``: equals ``mlstm_recurrent_sequence`` in
  float64 (the cell and ``native_sequence.py`` are the same recurrence; the
  cell's softplus-form log-sigmoid agrees with ``F.logsigmoid`` there), with and
  without a carried state.
* ``arbitrary_length``: equals the plain sequence loop for every S.
* ``mlstm_chunkwise_bw`` (the reference's custom backward): in float64 it equals
  torch.autograd through ``mlstm_chunkwise_fw`` wherever the reference's
  simplification is exact — a loss that depends on h only through each row's
  direction (h / |h|, what the layer's multi-head norm sees), with and without
  initial states (dq, dk, dv, di, df, dc0, dn0 = 0); and a loss
  <G, C_last exp(m_last)> on the last state, where dq, dk, dv, di and dc0 equal
  autograd's and df equals autograd's minus <G, C_last exp(m_last)> sigmoid(-f)
  (the constant the reference's suffix-sum formula for df leaves out on that
  path); it is invariant to the chunk size.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = [
    "recurrent_fw_C",
    "parallel_fw_H",
    "mlstm_chunkwise_fw",
    "mlstm_chunkwise",
    "mlstm_recurrent_kernel_cell",
    "mlstm_recurrent_step",
    "mlstm_recurrent_sequence",
    "mlstm_parallel_fw",
    "arbitrary_length",
    "mlstm_chunkwise_bw",
]


def recurrent_fw_C(matK, matV, vecB, vecI, matC_initial=None, vecN_initial=None,
                   scaM_initial=None, chunk_size=64, num_chunks=1):
    """Inter-chunk recurrence; materialises the NC+1 chunk-boundary states.

    Follows ``VTN/fw.py:29-145``: ``a = b_L - b + i`` (``:98``), ``g = b_L``
    (``:99``), per chunk ``m' = max(g + m, max a)`` (``:115``),
    ``Kbar = K exp(a - m')`` (``:121-123``), ``Gbar = exp(g + m - m')``
    (``:125``), ``C' = Gbar C + Kbar^T V`` (``:128-130``),
    ``n' = Gbar n + sum_t Kbar`` (``:133``).  States keep ``matK.dtype``
    (``:65,71-97``).
    """
    B, NH, S, DHQK = matK.shape
    DHV = matV.shape[-1]
    NC, L = num_chunks, chunk_size
    dt, dev = matK.dtype, matK.device
    C_states = torch.zeros((B, NH, (NC + 1) * DHQK, DHV), dtype=dt, device=dev)
    n_states = torch.zeros((B, NH, (NC + 1) * DHQK), dtype=dt, device=dev)
    m_states = torch.zeros((B, NH, NC + 1), dtype=dt, device=dev)

    C = matC_initial if matC_initial is not None else torch.zeros((B, NH, DHQK, DHV), dtype=dt, device=dev)
    n = vecN_initial if vecN_initial is not None else torch.zeros((B, NH, DHQK), dtype=dt, device=dev)
    m = scaM_initial if scaM_initial is not None else torch.zeros((B, NH, 1), dtype=dt, device=dev)
    m = m.squeeze(-1)

    vecA = vecB[..., -1, None] - vecB + vecI
    scaG = vecB[..., -1]
    scaA_max = vecA.max(-1).values

    for c in range(NC):
        C_states[:, :, c * DHQK:(c + 1) * DHQK, :] = C
        n_states[:, :, c * DHQK:(c + 1) * DHQK] = n
        m_states[:, :, c] = m
        m_next = torch.max(scaG[:, :, c] + m, scaA_max[:, :, c])
        Kc = matK[:, :, c * L:(c + 1) * L, :]
        Vc = matV[:, :, c * L:(c + 1) * L, :]
        Kbar = Kc * torch.exp(vecA[:, :, c, :] - m_next[..., None])[:, :, :, None]
        Gbar = torch.exp(scaG[:, :, c] + m - m_next)[:, :, None]
        C = Gbar[..., None] * C + Kbar.transpose(-2, -1) @ Vc
        n = Gbar * n + Kbar.transpose(-2, -1).sum(-1)
        m = m_next

    C_states[:, :, -DHQK:, :] = C
    n_states[:, :, -DHQK:] = n
    m_states[:, :, -1] = m
    return C_states, n_states, m_states


def parallel_fw_H(matQ, matK, matV, C_states, n_states, m_states, vecI, vecB,
                  qk_scale, chunk_size=64, num_chunks=1, eps=1e-6):
    """Intra-chunk outputs combined with the inter-chunk states.

    Follows ``VTN/fw.py:148-254``: ``logD_ij = b_i - b_j + i_j`` for j <= i
    else -inf (``:204-208``); ``m_intra = rowmax logD`` (``:211-213``);
    ``m = max(b + m_inter, m_intra)`` (``:216-217``); ``S = Q K^T s``
    (``:225``); ``M = S exp(logD - m)`` (``:222-227``);
    ``Qbar = Q exp(b + m_inter - m) s`` (``:230-231``);
    ``num = Qbar C + M V``, ``den = Qbar n + sum_j M`` (``:233-239``);
    ``h = num / (max(|den|, exp(-m)) + eps)`` (``:241-245``).
    Returns ``(h, max(|den|, exp(-m)), m)`` with shapes (B,NH,S,DHV),
    (B,NH,S), (B,NH,S).
    """
    B, NH, S, DHQK = matQ.shape
    DHV = matV.shape[-1]
    NC, L = num_chunks, chunk_size
    Ck = C_states.reshape(B, NH, NC, DHQK, DHV)
    nk = n_states.reshape(B, NH, NC, DHQK)
    Q = matQ.reshape(B, NH, NC, L, DHQK)
    K = matK.reshape(B, NH, NC, L, DHQK)
    V = matV.reshape(B, NH, NC, L, DHV)

    causal = torch.tril(torch.ones((L, L), dtype=torch.bool, device=matQ.device))
    logF = vecB[:, :, :, :, None] - vecB[:, :, :, None, :]
    logF = torch.where(causal, logF, -float("inf"))
    logD = logF + vecI[:, :, :, None, :]
    m_intra = torch.max(logD, dim=-1, keepdim=False).values
    m_b_inter = vecB + m_states[:, :, :, None]
    m_comb = torch.maximum(m_b_inter, m_intra)[..., None]
    m_b_inter = m_b_inter[..., None]

    D = torch.exp(logD - m_comb)
    Smat = (Q @ K.transpose(-2, -1)) * qk_scale
    M = Smat * D
    Bbar = torch.exp(m_b_inter - m_comb)
    Qbar = Q * Bbar * qk_scale
    num = Qbar @ Ck + M @ V
    den = Qbar @ nk.unsqueeze(-1) + M.sum(dim=-1, keepdim=True)
    den_max = torch.maximum(torch.abs(den), torch.exp(-m_comb))
    H = num / (den_max + eps)
    return (H.reshape(B, NH, S, DHV), den_max.reshape(B, NH, S), m_comb.reshape(B, NH, S))


def mlstm_chunkwise_fw(matQ, matK, matV, vecI, vecF, matC_initial=None, vecN_initial=None,
                       scaM_initial=None, qk_scale=None, return_last_states=False,
                       return_all_states=False, chunk_size=64, eps=1e-6):
    """Chunkwise mLSTM forward, ``VTN/fw.py:257-369``.

    Requires ``S % chunk_size == 0`` (``:303-305``); gates are
    ``b = cumsum(logsigmoid(f))`` per chunk (``:308-313``); ``qk_scale``
    defaults to ``DHQK ** -0.5`` (``:315-316``).  Returns
    ``(h, n_out, m_out, last_states | None, all_states | None)``.
    """
    B, NH, S, DHQK = matQ.shape
    assert S % chunk_size == 0, f"Sequence length {S} is not divisible by chunk size {chunk_size}."
    NC = S // chunk_size
    vecI = vecI.reshape(B, NH, NC, chunk_size)
    vecF = vecF.reshape(B, NH, NC, chunk_size)
    vecB = F.logsigmoid(vecF).cumsum(-1)
    if qk_scale is None:
        qk_scale = DHQK ** -0.5
    C_states, n_states, m_states = recurrent_fw_C(
        matK, matV, vecB, vecI, matC_initial, vecN_initial, scaM_initial,
        chunk_size=chunk_size, num_chunks=NC)
    H, n_out, m_out = parallel_fw_H(
        matQ, matK, matV, C_states[:, :, :-DHQK, :], n_states[:, :, :-DHQK],
        m_states[:, :, :-1], vecI, vecB, qk_scale, chunk_size=chunk_size,
        num_chunks=NC, eps=eps)
    last = None
    if return_last_states:
        last = (C_states[:, :, -DHQK:, :], n_states[:, :, -DHQK:], m_states[:, :, -1:])
    allst = (C_states, n_states, m_states) if return_all_states else None
    return H, n_out, m_out, last, allst


def mlstm_chunkwise(matQ, matK, matV, vecI, vecF, matC_initial=None, vecN_initial=None,
                    scaM_initial=None, qk_scale=None, return_last_states=False,
                    chunk_size=64, eps=1e-6):
    """Public chunkwise entry point, ``VTN/fw.py:372-412``."""
    H, _, _, last, _ = mlstm_chunkwise_fw(
        matQ, matK, matV, vecI, vecF, matC_initial, vecN_initial, scaM_initial,
        qk_scale=qk_scale, return_last_states=return_last_states,
        chunk_size=chunk_size, eps=eps)
    return (H, last) if return_last_states else H


def mlstm_recurrent_step(q, k, v, i, f, c, n, m, eps=1e-6, dtype_state=torch.float32, gate_exp=torch.exp):
    """One recurrent decode step, ``REC/native_step.py:8-133``.

    ``m' = max(logsigmoid(f) + m, i)`` (``:70-73``); ``fa = exp(logsig f + m
    - m')``, ``ia = exp(i - m')`` (``:75-76``); ``q_s = q DHQK^-0.5``
    (``:78``); ``C' = fa C + ia (k v^T)`` (``:79-81``); ``n' = fa n + ia k``
    (``:82``); ``h = q_s C'.to(q.dtype) / (max(|q_s n'.to(q.dtype)|,
    exp(-m')) + eps)`` (``:83-96``).  h is returned in q's dtype and the
    states in ``dtype_state`` (``:98-101``).  ``gate_exp`` computes the three
    exponentials (fa, ia, exp(-m')); tests pass a perturbed one to measure how
    far the reference's roundings move h under 1-ulp changes of them.
    """
    dtype_qkv = q.dtype
    C_old = c.to(dtype=dtype_state)
    n_old = n.to(dtype=dtype_state)
    m_old = m.to(dtype=dtype_state)
    B, NH, DHQK = q.shape
    lsf = F.logsigmoid(f)
    m_new = torch.max(lsf + m_old, i)
    fa = gate_exp(lsf + m_old - m_new)
    ia = gate_exp(i - m_new)
    q_s = q * (DHQK ** (-0.5))
    C_new = fa[:, :, :, None] * C_old + ia[:, :, :, None] * (k[:, :, :, None] @ v[:, :, None, :])
    n_new = fa * n_old + ia * k
    h_num = (q_s[:, :, None, :] @ C_new.to(dtype=dtype_qkv)).squeeze(2).to(dtype=dtype_state)
    qn = (q_s[:, :, None, :] @ n_new[:, :, :, None].to(dtype=dtype_qkv)).squeeze(2)
    h_den = (torch.maximum(qn.abs(), gate_exp(-m_new)) + eps).to(dtype=dtype_state)
    h = (h_num / h_den).to(dtype=dtype_qkv)
    return h, (C_new.to(dtype=dtype_state), n_new.to(dtype=dtype_state), m_new.to(dtype=dtype_state))


def mlstm_recurrent_sequence(q, k, v, i, f, c_initial=None, n_initial=None, m_initial=None,
                             return_last_states=False, eps=1e-6, dtype_state=torch.float32, gate_exp=torch.exp):
    """Time loop over :func:`mlstm_recurrent_step`, ``REC/native_sequence.py:18-170``.

    Zero initial states (m = 0) when none are given (``:63-69``).
    """
    B, NH, S, DHQK = q.shape
    DHV = v.shape[-1]
    if c_initial is not None:
        assert n_initial is not None and m_initial is not None, "Initial states must be provided together."
        C, n, m = c_initial.to(dtype_state), n_initial.to(dtype_state), m_initial.to(dtype_state)
    else:
        C = torch.zeros((B, NH, DHQK, DHV), dtype=dtype_state, device=q.device)
        n = torch.zeros((B, NH, DHQK), dtype=dtype_state, device=q.device)
        m = torch.zeros((B, NH, 1), dtype=dtype_state, device=q.device)
    hs = []
    for t in range(S):
        h, (C, n, m) = mlstm_recurrent_step(
            q[:, :, t, :], k[:, :, t, :], v[:, :, t, :], i[:, :, t, None], f[:, :, t, None],
            C, n, m, eps=eps, dtype_state=dtype_state, gate_exp=gate_exp)
        hs.append(h)
    H = torch.stack(hs, dim=-2)
    return (H, (C, n, m)) if return_last_states else H


def mlstm_recurrent_kernel_cell(q, k, v, i, f, state=None, eps=1e-6):
    """``mLSTMRecurrentKernelCell.forward`` (``xlstm_metal/torch_native/blocks/mlstm/mlstm_chunkwise/
    mlstm_recurrent_kernel_cell.py:53-161``) with its default float32 compute and state dtypes.

    q, k [B, NH, S, DHQK], v [B, NH, S, DHV], i, f [B, NH, S]; state (C, n, m [B, NH]) or None
    (zeros, ``:99-102``).  Per step: ``f_log = -log(1 + exp(-f))`` (``:129``, the softplus form,
    not ``F.logsigmoid``), ``m' = max(f_log + m, i)``, ``fg = exp(f_log + m - m')``, ``ig = exp(i -
    m')`` (``:130-134``), ``C' = fg C + ig k v^T``, ``n' = fg n + ig k`` (``:138-146``), ``q_s = q
    rsqrt(DHQK)`` (``:152``), ``h = sum(C' q_s) / (max(|n' . q_s|, exp(-m')) + eps)``
    (``:155-163``).  Returns (h [B, NH, S, DHV], (C, n, m [B, NH])).
    """
    B, NH, S, DHQK = q.shape
    DHV = v.shape[-1]
    dt = q.dtype
    if state is None:
        C = torch.zeros((B, NH, DHQK, DHV), dtype=dt)
        n = torch.zeros((B, NH, DHQK), dtype=dt)
        m = torch.zeros((B, NH), dtype=dt)
    else:
        C, n, m = (t.to(dt) for t in state)
    hs = []
    for t in range(S):
        q_t, k_t, v_t, i_t, f_t = q[:, :, t], k[:, :, t], v[:, :, t], i[:, :, t], f[:, :, t]
        f_log = -torch.log(1.0 + torch.exp(-f_t))
        m_new = torch.maximum(f_log + m, i_t)
        fg = torch.exp(f_log + m - m_new)
        ig = torch.exp(i_t - m_new)
        C = fg[:, :, None, None] * C + ig[:, :, None, None] * (k_t[:, :, :, None] * v_t[:, :, None, :])
        n = fg[:, :, None] * n + ig[:, :, None] * k_t
        m = m_new
        q_s = q_t * DHQK ** -0.5
        h_num = (C * q_s[:, :, :, None]).sum(dim=2)
        qn = (n * q_s).sum(dim=2, keepdim=True)
        h_den = torch.maximum(qn.abs(), torch.exp(-m)[:, :, None]) + eps
        hs.append(h_num / h_den)
    return torch.stack(hs, dim=2), (C, n, m)


def mlstm_parallel_fw(matQ, matK, matV, vecI, vecF, eps=1e-6):
    """Quadratic (fully parallel) stabilised form, ``PV/torch_native/fw.py:15-74``.

    Its row max omits the zero initial-state term, so it equals the chunkwise
    form exactly when ``eps = 0`` and to within ``eps * exp(m)`` otherwise.
    Returns ``(h, n, m)``.
    """
    B, NH, S, DHQK = matQ.shape
    lsf = F.logsigmoid(vecF)
    cum = lsf[:, :, :, None].repeat(1, 1, 1, S).tril(-1).cumsum(-2)
    causal = torch.tril(torch.ones((S, S), dtype=torch.bool, device=matQ.device))
    logD = torch.where(causal, cum, -float("inf")) + vecI[:, :, None, :]
    m, _ = torch.max(logD, dim=-1, keepdim=True)
    D = torch.exp(logD - m)
    Smat = (matQ @ matK.transpose(-2, -1)) * (DHQK ** -0.5)
    Ct = Smat * D
    nrm = torch.maximum(Ct.sum(dim=-1, keepdim=True).abs(), torch.exp(-m))
    H = (Ct / (nrm + eps)) @ matV
    return H, nrm.squeeze(-1), m.squeeze(-1)


def arbitrary_length(q, k, v, f, i, c_initial=None, n_initial=None, m_initial=None,
                     return_last_states=True, eps=1e-6, chunk_size=64, dtype_state=torch.float32):
    """Any-S inference driver, ``PT/kernel_wrappers.py:12-202``.

    Tries chunk sizes ``chunk_size, chunk_size/2, ...`` down to 16 (``:74-78``),
    runs the chunkwise form on the largest whole number of chunks at each size
    carrying (C, n, m) (``:107-149``), finishes a tail shorter than 16 with the
    sequence loop (``:151-170``) and calls the single step when S == 1
    (``:173-197``).  Zero states are float32 (``:84-98``).  ``dtype_state`` is
    the state dtype the step and sequence kernels are bound with
    (``PT/backend_module.py:103-113``).
    """
    B, NH, S, DHQK = k.shape
    DHV = v.shape[-1]
    sizes = []
    cs = chunk_size
    while cs >= 16:
        sizes.append(cs)
        cs //= 2
    C = c_initial if c_initial is not None else torch.zeros(B, NH, DHQK, DHV, dtype=torch.float32)
    n = n_initial if n_initial is not None else torch.zeros(B, NH, DHQK, dtype=torch.float32)
    m = m_initial if m_initial is not None else torch.zeros(B, NH, 1, dtype=torch.float32)
    if S > 1:
        outs = []
        start = 0
        for cs in sizes:
            rem = S - start
            if rem < cs:
                continue
            end = start + cs * (rem // cs)
            h, (C, n, m) = mlstm_chunkwise(
                q[..., start:end, :], k[..., start:end, :], v[..., start:end, :],
                i[..., start:end], f[..., start:end], C, n, m,
                return_last_states=True, chunk_size=cs, eps=eps)
            outs.append(h)
            start = end
            if rem % cs == 0:
                break
        if S - start > 0:
            h, (C, n, m) = mlstm_recurrent_sequence(
                q[..., start:, :], k[..., start:, :], v[..., start:, :], i[..., start:],
                f[..., start:], C, n, m, return_last_states=True, eps=eps, dtype_state=dtype_state)
            outs.append(h)
        H = torch.cat(outs, dim=2)
    else:
        assert S == 1, f"Received empty sequence (S={S}), require at least single element in the sequence."
        h, (C, n, m) = mlstm_recurrent_step(q.squeeze(2), k.squeeze(2), v.squeeze(2), i, f, C, n, m, eps=eps,
                                            dtype_state=dtype_state)
        H = h[:, :, None, :]
    return (H, (C, n, m)) if return_last_states else H


def mlstm_chunkwise_bw(matQ, matK, matV, vecI, vecF, matDeltaH, matC_initial=None, vecN_initial=None,
                       scaM_initial=None, matDeltaC_last=None, qk_scale=None, chunk_size=64, eps=1e-6,
                       state_round=None):
    """The reference's custom chunkwise backward, ``VTN/bw.py:198-352``.

    States are recomputed from the inputs (``:242-258``) and the forward's
    per-token divisor ``N = max(|den|, exp(-m))`` and stabiliser ``m`` are taken
    as constants (``:44-47``).  Reverse recurrence (``:31-115``):
    ``dC_{c} = exp(g_c + m_c - m_{c+1}) dC_{c+1} + Qbar_c^T (dH_c / (N_c + eps))``
    with ``Qbar = Q exp(b + m_c - m) s``.  Per chunk (``:118-195``):
    ``Dbar = exp(logD - m)``, ``Sbar = Q K^T s Dbar``, ``dS = (dH~ V^T) Dbar``,
    ``dV = Sbar^T dH~ + (K Abar) dC_{c+1}``, ``dK = dS^T Q s + (V Abar) dC_{c+1}^T``,
    ``dQ = dS K s + (dH~ Bbar) (C_c s)^T`` with ``Abar = exp(b_L - b + i - m_{c+1})``,
    ``Bbar = exp(b + m_c - m)``.  Gates (``:330-338``): ``dF = sigmoid(-f)`` times the
    suffix sum over the sequence of ``sum_d (q dq - k dk)``, ``dI = sum_d v dv``.
    Returns ``(dq, dk, dv, di, df, dc0 | None, dn0 | None, dm0 | None)``; dn0 and dm0
    are zeros, as there (``:340-342``).  ``state_round`` (tests only), if given, is applied to
    the per-chunk states C and dC where the per-chunk products consume them, to model a storage
    format of the materialised states.
    """
    B, NH, S, DHQK = matQ.shape
    DHV = matV.shape[-1]
    L = chunk_size
    assert S % L == 0, f"Sequence length {S} is not divisible by chunk size {L}."
    NC = S // L
    if qk_scale is None:
        qk_scale = DHQK ** -0.5
    vecB = F.logsigmoid(vecF.reshape(B, NH, NC, L)).cumsum(-1)
    vecIr = vecI.reshape(B, NH, NC, L)
    C_states, n_states, m_states = recurrent_fw_C(matK, matV, vecB, vecIr, matC_initial, vecN_initial,
                                                  scaM_initial, chunk_size=L, num_chunks=NC)
    _, n_out, m_out = parallel_fw_H(matQ, matK, matV, C_states[:, :, :-DHQK, :], n_states[:, :, :-DHQK],
                                    m_states[:, :, :-1], vecIr, vecB, qk_scale, chunk_size=L, num_chunks=NC,
                                    eps=eps)
    Cs = C_states.reshape(B, NH, NC + 1, DHQK, DHV)
    if state_round is not None:
        Cs = state_round(Cs)
    dH_t = matDeltaH / (n_out + eps)[..., None]  # dH~, (B, NH, S, DHV)

    def chunk(x, c):
        return x[:, :, c * L:(c + 1) * L]

    # reverse recurrence over the chunks
    g = vecB[..., -1]
    dC = (matDeltaC_last.to(matQ.dtype) if matDeltaC_last is not None
          else torch.zeros((B, NH, DHQK, DHV), dtype=matQ.dtype, device=matQ.device))
    dC_after = [None] * NC  # gradient of the state after chunk c
    for c in range(NC - 1, -1, -1):
        dC_after[c] = dC if state_round is None else state_round(dC)
        m_c, m_n = m_states[:, :, c], m_states[:, :, c + 1]
        gbar = torch.exp(g[:, :, c] + m_c - m_n)[:, :, None, None]
        bbar = torch.exp(vecB[:, :, c] + m_c[..., None] - chunk(m_out, c))[..., None]
        Qbar = chunk(matQ, c) * bbar * qk_scale
        dC = gbar * dC + Qbar.transpose(-2, -1) @ chunk(dH_t, c)
    dC_initial = dC

    causal = torch.tril(torch.ones((L, L), dtype=torch.bool, device=matQ.device))
    dQ, dK, dV = torch.empty_like(matQ), torch.empty_like(matK), torch.empty_like(matV)
    for c in range(NC):
        Qc, Kc, Vc, dHc = chunk(matQ, c), chunk(matK, c), chunk(matV, c), chunk(dH_t, c)
        b, ic, mc = vecB[:, :, c], vecIr[:, :, c], chunk(m_out, c)
        m_c, m_n = m_states[:, :, c], m_states[:, :, c + 1]
        logD = torch.where(causal, b[..., :, None] - b[..., None, :], -float("inf")) + ic[..., None, :]
        Dbar = torch.exp(logD - mc[..., None])
        Sbar = (Qc @ Kc.transpose(-2, -1)) * qk_scale * Dbar
        dS = (dHc @ Vc.transpose(-2, -1)) * Dbar
        Abar = torch.exp(b[..., -1:] - b + ic - m_n[..., None])[..., None]
        Bbar = torch.exp(b + m_c[..., None] - mc)[..., None]
        dV[:, :, c * L:(c + 1) * L] = Sbar.transpose(-2, -1) @ dHc + (Kc * Abar) @ dC_after[c]
        dK[:, :, c * L:(c + 1) * L] = (dS.transpose(-2, -1) @ Qc) * qk_scale + (Vc * Abar) @ dC_after[c].transpose(-2, -1)
        dQ[:, :, c * L:(c + 1) * L] = (dS @ Kc) * qk_scale + (dHc * Bbar) @ (Cs[:, :, c] * qk_scale).transpose(-2, -1)

    per_token = (matQ * dQ - matK * dK).sum(-1)
    suffix = per_token.flip(-1).cumsum(-1).flip(-1)
    dF = suffix * torch.sigmoid(-vecF)
    dI = (matV * dV).sum(-1)
    dc0 = dC_initial if matC_initial is not None else None
    dn0 = torch.zeros_like(vecN_initial) if vecN_initial is not None else None
    dm0 = torch.zeros_like(scaM_initial) if scaM_initial is not None else None
    return dQ, dK, dV, dI, dF, dc0, dn0, dm0
