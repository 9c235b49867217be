"""Element-by-element pure-Python versions of the hot path for tiny inputs — the
independent pins of oracle.reference and oracle.csr (test infrastructure, see
oracle/__init__.py). Everything is float64 from the given (already rounded) inputs.
"""


def encode(x, W_enc, b_enc, b_dec, threshold=None, activation="relu", k=None):
    """act(sum_i (x[m][i] - b_dec[i]) * W_enc[i][n] + b_enc[n])  (reference.py:36-46)."""
    M, K, N = len(x), len(W_enc), len(W_enc[0])
    pre = [[b_enc[n] + sum((x[m][i] - b_dec[i]) * W_enc[i][n] for i in range(K)) for n in range(N)]
           for m in range(M)]
    out = []
    for m in range(M):
        if activation == "relu":
            out.append([max(p, 0.0) for p in pre[m]])
        elif activation == "jumprelu":
            out.append([max(p, 0.0) if p > threshold[n] else 0.0 for n, p in enumerate(pre[m])])
        else:  # topk of pre, then relu of the kept values (reference.py:45-46)
            keep = sorted(range(N), key=lambda n: (-pre[m][n], n))[:k]
            row = [0.0] * N
            for n in keep:
                row[n] = max(pre[m][n], 0.0)
            out.append(row)
    return pre, out


def dense_to_csr(f):
    """Canonical CSR by scanning each row left to right (decode.py:61-74)."""
    indptr, indices, values = [0], [], []
    for row in f:
        for n, v in enumerate(row):
            if v != 0:
                indices.append(n)
                values.append(v)
        indptr.append(len(indices))
    return indptr, indices, values


def sparse_decode(indptr, indices, values, W_dec, b_dec=None):
    """x_hat[m][d] = b_dec[d] + sum_j values[j] * W_dec[indices[j]][d]  (decode.py:42-55)."""
    D = len(W_dec[0])
    out = []
    for m in range(len(indptr) - 1):
        row = [b_dec[d] if b_dec is not None else 0.0 for d in range(D)]
        for j in range(indptr[m], indptr[m + 1]):
            for d in range(D):
                row[d] += values[j] * W_dec[indices[j]][d]
        out.append(row)
    return out


def topk(f, k):
    """Per row: the k (value, column) pairs with the largest values; ties by lower column."""
    vals, cols = [], []
    for row in f:
        order = sorted(range(len(row)), key=lambda n: (-row[n], n))[:k]
        vals.append([row[n] for n in order])
        cols.append(order)
    return vals, cols
