function initstacks_binsum_b()
    return nothing
end

function binsum_b(loss, lossb, v, vb, bins, c, cb, i_n, i_b)
    for i = 1:i_n
        c[bins[i]] = c[bins[i]] + v[i] ^ 2
    end
    for b = 1:i_b
        loss[1] = loss[1] + c[b] ^ 2
    end
    for b = i_b:-1:1
        cb[b] = cb[b] + 2 * c[b] * lossb[1]
    end
    for i = i_n:-1:1
        __icse_0 = bins[i]
        vb[i] = vb[i] + 2 * v[i] * cb[__icse_0]
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
