function binsum_d(loss, lossd, v, vd, bins, c, cd, i_n, i_b)
    for i = 1:i_n
        __icse_0 = bins[i]
        cd[__icse_0] = cd[__icse_0] + 2 * v[i] * vd[i]
        c[__icse_0] = c[__icse_0] + v[i] ^ 2
    end
    for b = 1:i_b
        lossd[1] = lossd[1] + 2 * c[b] * cd[b]
        loss[1] = loss[1] + c[b] ^ 2
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
