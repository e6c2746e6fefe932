function initstacks_binsum_b()
    return nothing
end

function binsum_hv(loss, lossb, v, vb, bins, c, cb, i_n, i_b, lossd, lossbd, vd, vbd, cd, cbd)
    for i = 1:i_n
        __icse_0 = bins[i]
        cd[__icse_0] = cd[__icse_0] + 2 * v[i] * vd[i]
        c[__icse_0] = c[__icse_0] + v[i] ^ 2
    end
    for b = 1:i_b
        lossd[1] = lossd[1] + 2 * c[b] * cd[b]
        loss[1] = loss[1] + c[b] ^ 2
    end
    for b = i_b:-1:1
        cbd[b] = cbd[b] + (2 * cd[b] * lossb[1] + 2 * c[b] * lossbd[1])
        cb[b] = cb[b] + 2 * c[b] * lossb[1]
    end
    for i = i_n:-1:1
        __icse_1 = bins[i]
        vbd[i] = vbd[i] + (2 * vd[i] * cb[__icse_1] + 2 * v[i] * cbd[__icse_1])
        vb[i] = vb[i] + 2 * v[i] * cb[__icse_1]
    end
    return nothing
end

function binsum(loss, v, bins, c, i_n, i_b)
    for i = 1:i_n
        c[bins[i]] = c[bins[i]] + v[i] ^ 2
    end
    for b = 1:i_b
        loss[1] = loss[1] + c[b] ^ 2
    end
    return nothing
end
