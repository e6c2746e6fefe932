function initstacks_diffusion2d_b()
    return nothing
end

function diffusion2d_hv(loss, lossb, u, ub, un, unb, n, lossd, lossbd, ud, ubd, und, unbd)
    for idx = 1:n * n
        __icse_0 = idx - 1
        i = mod(__icse_0, n) + 1
        j = div(__icse_0, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        __icse_1 = (j - 1) * n
        und[idx] = ud[idx] + 0.1 * ((((ud[__icse_1 + im] + ud[__icse_1 + ip]) + ud[(jm - 1) * n + i]) + ud[(jp - 1) * n + i]) + -(4.0 * ud[idx]))
        un[idx] = u[idx] + 0.1 * (u[__icse_1 + im] + u[__icse_1 + ip] + u[(jm - 1) * n + i] + u[(jp - 1) * n + i] - 4.0 * u[idx])
    end
    for k = 1:n * n
        __hcse_2 = un[k]
        lossd[1] = lossd[1] + (2__hcse_2) * und[k]
        loss[1] = loss[1] + __hcse_2 ^ 2
    end
    for k = n * n:-1:1
        __hcse_3 = lossb[1]
        __hcse_4 = 2 * un[k]
        unbd[k] = unbd[k] + (__hcse_3 * (2 * und[k]) + __hcse_4 * lossbd[1])
        unb[k] = unb[k] + __hcse_4 * __hcse_3
    end
    for idx = n * n:-1:1
        __icse_5 = idx - 1
        i = mod(__icse_5, n) + 1
        j = div(__icse_5, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        __oldb_0d = unbd[idx]
        __oldb_0 = unb[idx]
        unbd[idx] = 0.0
        unb[idx] = 0.0
        ubd[idx] = ubd[idx] + __oldb_0d
        ub[idx] = ub[idx] + __oldb_0
        __cse_6d = 0.1__oldb_0d
        __cse_6 = 0.1__oldb_0
        __icse_7 = (j - 1) * n
        ubd[__icse_7 + im] = ubd[__icse_7 + im] + __cse_6d
        ub[__icse_7 + im] = ub[__icse_7 + im] + __cse_6
        ubd[__icse_7 + ip] = ubd[__icse_7 + ip] + __cse_6d
        ub[__icse_7 + ip] = ub[__icse_7 + ip] + __cse_6
        ubd[(jm - 1) * n + i] = ubd[(jm - 1) * n + i] + __cse_6d
        ub[(jm - 1) * n + i] = ub[(jm - 1) * n + i] + __cse_6
        ubd[(jp - 1) * n + i] = ubd[(jp - 1) * n + i] + __cse_6d
        ub[(jp - 1) * n + i] = ub[(jp - 1) * n + i] + __cse_6
        ubd[idx] = ubd[idx] + 4.0 * -__cse_6d
        ub[idx] = ub[idx] + 4.0 * -__cse_6
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
