function initstacks_diffusion2d_b()
    return nothing
end

function diffusion2d_b(loss, lossb, u, ub, un, unb, n)
    for idx = 1:n * n
        __icse_0 = idx - 1
        i = mod(__icse_0, n) + 1
        j = div(__icse_0, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        __icse_1 = (j - 1) * n
        un[idx] = u[idx] + 0.1 * (u[__icse_1 + im] + u[__icse_1 + ip] + u[(jm - 1) * n + i] + u[(jp - 1) * n + i] - 4.0 * u[idx])
    end
    for k = 1:n * n
        loss[1] = loss[1] + un[k] ^ 2
    end
    for k = n * n:-1:1
        unb[k] = unb[k] + (2 * un[k]) * lossb[1]
    end
    for idx = n * n:-1:1
        __icse_2 = idx - 1
        i = mod(__icse_2, n) + 1
        j = div(__icse_2, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        __oldb_0 = unb[idx]
        unb[idx] = 0.0
        ub[idx] = ub[idx] + __oldb_0
        __cse_3 = 0.1__oldb_0
        __icse_4 = (j - 1) * n
        ub[__icse_4 + im] = ub[__icse_4 + im] + __cse_3
        ub[__icse_4 + ip] = ub[__icse_4 + ip] + __cse_3
        ub[(jm - 1) * n + i] = ub[(jm - 1) * n + i] + __cse_3
        ub[(jp - 1) * n + i] = ub[(jp - 1) * n + i] + __cse_3
        ub[idx] = ub[idx] + 4.0 * -__cse_3
    end
    return nothing
end

function diffusion2d(loss, u, un, n)
    for idx = 1:n * n
        i = mod(idx - 1, n) + 1
        j = div(idx - 1, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        un[idx] = u[idx] + 0.1 * (u[(j - 1) * n + im] + u[(j - 1) * n + ip] + u[(jm - 1) * n + i] + u[(jp - 1) * n + i] - 4.0 * u[idx])
    end
    for k = 1:n * n
        loss[1] = loss[1] + un[k] ^ 2
    end
    return nothing
end
