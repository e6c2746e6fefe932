function initstacks_window1d_b()
    return nothing
end

function window1d_b(loss, lossb, inp, inpb, w, wb, out, outb, i_n, i_k)
    s = 0.0
    sb = 0.0
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
    for q = i_n - i_k + 1:-1:1
        outb[q] = outb[q] + 0.5 * (2 * out[q]) * lossb[1]
    end
    for i = i_n - i_k + 1:-1:1
        __oldb_0 = outb[i]
        outb[i] = 0.0
        sb = sb + __oldb_0
        for k = i_k:-1:1
            __icse_0 = i + k - 1
            wb[k] = wb[k] + inp[__icse_0] * sb
            inpb[__icse_0] = inpb[__icse_0] + w[k] * sb
        end
        sb = 0.0
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
