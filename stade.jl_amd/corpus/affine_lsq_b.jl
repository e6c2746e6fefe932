function initstacks_affine_lsq_b()
    return nothing
end

function affine_lsq_b(loss, lossb, w, wb, x, xb, b, bb, t, tb, r, rb, i_m, i_n)
    s = 0.0
    sb = 0.0
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
    for i_i2 = i_m:-1:1
        rb[i_i2] = rb[i_i2] + 0.5 * (2 * r[i_i2]) * lossb[1]
    end
    for i_i = i_m:-1:1
        __oldb_0 = rb[i_i]
        rb[i_i] = 0.0
        sb = sb + __oldb_0
        for i_j = i_n:-1:1
            wb[i_i, i_j] = wb[i_i, i_j] + x[i_j] * sb
            xb[i_j] = xb[i_j] + w[i_i, i_j] * sb
        end
        __oldb_1 = sb
        sb = 0.0
        bb[i_i] = bb[i_i] + __oldb_1
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
