function initstacks_affine_lsq_b()
    return nothing
end

function affine_lsq_hv(loss, lossb, w, wb, x, xb, b, bb, t, tb, r, rb, i_m, i_n, lossd, lossbd, wd, wbd, xd, xbd, bd, bbd, td, tbd, rd, rbd)
    s = 0.0
    sd = 0.0
    sb = 0.0
    sbd = 0.0
    for i_i = 1:i_m
        sd = bd[i_i] - td[i_i]
        s = b[i_i] - t[i_i]
        for i_j = 1:i_n
            __hcse_0 = x[i_j]
            __hcse_1 = w[i_i, i_j]
            sd = sd + (__hcse_0 * wd[i_i, i_j] + __hcse_1 * xd[i_j])
            s = s + __hcse_1 * __hcse_0
        end
        rd[i_i] = sd
        r[i_i] = s
    end
    for i_i2 = 1:i_m
        __hcse_2 = r[i_i2]
        lossd[1] = lossd[1] + 0.5 * ((2__hcse_2) * rd[i_i2])
        loss[1] = loss[1] + 0.5 * __hcse_2 ^ 2
    end
    for i_i2 = i_m:-1:1
        __hcse_3 = lossb[1]
        __hcse_4 = 0.5 * (2 * r[i_i2])
        rbd[i_i2] = rbd[i_i2] + (__hcse_3 * (0.5 * (2 * rd[i_i2])) + __hcse_4 * lossbd[1])
        rb[i_i2] = rb[i_i2] + __hcse_4 * __hcse_3
    end
    for i_i = i_m:-1:1
        __oldb_0d = rbd[i_i]
        __oldb_0 = rb[i_i]
        rbd[i_i] = 0.0
        rb[i_i] = 0.0
        sbd = sbd + __oldb_0d
        sb = sb + __oldb_0
        for i_j = i_n:-1:1
            __hcse_5 = x[i_j]
            wbd[i_i, i_j] = wbd[i_i, i_j] + (sb * xd[i_j] + __hcse_5 * sbd)
            wb[i_i, i_j] = wb[i_i, i_j] + __hcse_5 * sb
            __hcse_6 = w[i_i, i_j]
            xbd[i_j] = xbd[i_j] + (sb * wd[i_i, i_j] + __hcse_6 * sbd)
            xb[i_j] = xb[i_j] + __hcse_6 * sb
        end
        __oldb_1d = sbd
        __oldb_1 = sb
        sbd = 0.0
        sb = 0.0
        bbd[i_i] = bbd[i_i] + __oldb_1d
        bb[i_i] = bb[i_i] + __oldb_1
        tbd[i_i] = tbd[i_i] + -__oldb_1d
        tb[i_i] = tb[i_i] + -__oldb_1
    end
    return nothing
end

function affine_lsq(loss, w, x, b, t, r, i_m, i_n)
    for i_i = 1:i_m
        s = b[i_i] - t[i_i]
        for i_j = 1:i_n
            s = s + w[i_i, i_j] * x[i_j]
        end
        r[i_i] = s
    end
    for i_i2 = 1:i_m
        loss[1] = loss[1] + 0.5 * r[i_i2] ^ 2
    end
    return nothing
end
