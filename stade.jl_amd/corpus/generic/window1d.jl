# window1d(loss, inp, w, out, i_n, i_k)
#
# A 1-D correlation with overlapping windows, out[i] = sum_k w[k] inp[i + k - 1] for the
# i_n - i_k + 1 full windows, then loss += 0.5 * sum(out .^ 2).  Its adjoint scatters into
# inp through overlapping windows and accumulates the i_k taps of wb from every window.
#
# loss: length-1 output, accumulated; inp: length i_n; w: length i_k;
# out: length i_n - i_k + 1, overwritten; i_n, i_k: lengths
function window1d(loss, inp, w, out, i_n, i_k)
    for i = 1:i_n - i_k + 1
        s = 0.0
        for k = 1:i_k
            s = s + w[k] * inp[i + k - 1]
        end
        out[i] = s
    end
    for q = 1:i_n - i_k + 1
        loss[1] = loss[1] + 0.5 * out[q] ^ 2
    end
    return nothing
end
