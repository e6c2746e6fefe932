function initstacks_window1d_b()
    return nothing
end

function window1d_hv(loss, lossb, inp, inpb, w, wb, out, outb, i_n, i_k, lossd, lossbd, inpd, inpbd, wd, wbd, outd, outbd)
    s = 0.0
    sb = 0.0
    sd = 0.0
    sbd = 0.0
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
    for q = i_n - i_k + 1:-1:1
        outbd[q] = outbd[q] + (0.5 * (2 * outd[q]) * lossb[1] + 0.5 * (2 * out[q]) * lossbd[1])
        outb[q] = outb[q] + 0.5 * (2 * out[q]) * lossb[1]
    end
    for i = i_n - i_k + 1:-1:1
        __oldb_0 = outb[i]
        __oldbd_0 = outbd[i]
        outb[i] = 0.0
        outbd[i] = 0.0
        sb = sb + __oldb_0
        sbd = sbd + __oldbd_0
        for k = i_k:-1:1
            __icse_0 = i + k - 1
            wbd[k] = wbd[k] + (inpd[__icse_0] * sb + inp[__icse_0] * sbd)
            wb[k] = wb[k] + inp[__icse_0] * sb
            inpbd[__icse_0] = inpbd[__icse_0] + (wd[k] * sb + w[k] * sbd)
            inpb[__icse_0] = inpb[__icse_0] + w[k] * sb
        end
        sb = 0.0
        sbd = 0.0
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
