function window1d_d(loss, lossd, inp, inpd, w, wd, out, outd, i_n, i_k)
    s = 0.0
    sd = 0.0
    for i = 1:i_n - i_k + 1
        sd = 0.0
        s = 0.0
        for k = 1:i_k
            sd = sd + (wd[k] * inp[i + k - 1] + w[k] * inpd[i + k - 1])
            s = s + w[k] * inp[i + k - 1]
        end
        outd[i] = sd
        out[i] = s
    end
    for q = 1:i_n - i_k + 1
        lossd[1] = lossd[1] + 0.5 * (2 * out[q]) * outd[q]
        loss[1] = loss[1] + 0.5 * out[q] ^ 2
    end
    return nothing
end

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
