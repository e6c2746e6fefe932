function affine_lsq_d(loss, lossd, w, wd, x, xd, b, bd, t, td, r, rd, i_m, i_n)
    for i_i = 1:i_m
        sd = bd[i_i] - td[i_i]
        s = b[i_i] - t[i_i]
        for i_j = 1:i_n
            __cse_0 = x[i_j]
            __cse_1 = w[i_i, i_j]
            sd = sd + (__cse_0 * wd[i_i, i_j] + __cse_1 * xd[i_j])
            s = s + __cse_1 * __cse_0
        end
        rd[i_i] = sd
        r[i_i] = s
    end
    for i_i2 = 1:i_m
        __cse_2 = r[i_i2]
        lossd[1] = lossd[1] + 0.5 * ((2__cse_2) * rd[i_i2])
        loss[1] = loss[1] + 0.5 * __cse_2 ^ 2
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
